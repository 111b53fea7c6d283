// Damped Cholesky chain (GPTQPlus._compute_hessian_inverse_with_fallback,
// gptq_utils/gptq_plus_utils.py:494-561) and the GPTQ+ first-order terms
// (_compute_gradient_terms :563-578, compute_safe_beta_from_reference_loss :174-194).
//
// The reference computes chol(H) -> cholesky_inverse -> chol(H^-1, upper) in fp32.  Here the
// upper factor U of H^-1 (U^T U = H^-1) is obtained with ONE factorisation: with P the
// index-reversal permutation and L L^T = P H P,  U = P L^-1 P.  The factorisation and the
// inverse L^-1 run together in one right-looking blocked pass in fp64 (64-wide panels):
//   per panel k:  L_kk = chol(A_kk) and T = L_kk^-1 in LDS (one workgroup),
//                 L_ik = A_ik T^T,  X_k = T B_k  (row block k of L^-1),
//                 A_ij -= L_ik L_jk^T (lower tiles),  B_i -= L_ik X_k   (fp64 MFMA GEMMs),
// where B accumulates I - sum_m L_im X_m.  H^-1 itself (Hinv_init) is P (L^-T L^-1) P and is
// only formed when asked for.  A non-positive or non-finite pivot, or a non-finite result,
// raises the device `info` flag; later kernels of the same attempt exit early.
#include "gemm_tile.h"

namespace {

constexpr int NB = 64;

__global__ void k_fill_i32(int* p, int v) { *p = v; }
__global__ void k_fill_f32(float* p, float v) { *p = v; }

// H_work[i,i] += fl32(p) * mean(diag(H_work)).  One workgroup.
__global__ __launch_bounds__(256) void k_damp(float* __restrict__ H, int C, float p) {
  __shared__ double part[256];
  double s = 0.0;
  for (int i = threadIdx.x; i < C; i += 256) s += (double)H[(int64_t)i * C + i];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) part[threadIdx.x] += part[threadIdx.x + o];
    __syncthreads();
  }
  const float mean = (float)(part[0] / (double)C);
  const float damp = p * mean;
  for (int i = threadIdx.x; i < C; i += 256) {
    float* d = H + (int64_t)i * C + i;
    *d = *d + damp;
  }
}

// A = P H_work P in fp64 (full square), Linv = 0.
__global__ __launch_bounds__(256) void k_reverse_to_f64(const float* __restrict__ H, int C,
                                                        double* __restrict__ A,
                                                        double* __restrict__ Linv) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= C) return;
  for (int i = blockIdx.y; i < C; i += gridDim.y) {
    A[(int64_t)i * C + j] = (double)H[(int64_t)(C - 1 - i) * C + (C - 1 - j)];
    Linv[(int64_t)i * C + j] = 0.0;
  }
}

// Factor the nb x nb diagonal block of A at (k, k) and invert it.  One workgroup.
// Writes T = L_kk^-1 (lower, explicit zeros above) to Tbuf and to Linv's diagonal block.
__global__ __launch_bounds__(256) void k_chol_diag(const double* __restrict__ A, int C, int k,
                                                   int nb, double* __restrict__ Tbuf,
                                                   double* __restrict__ Linv, int* info) {
  __shared__ double L[NB][NB + 1];
  __shared__ double T[NB][NB + 1];
  __shared__ int fail;
  if (*info) return;
  const int tid = threadIdx.x;
  if (tid == 0) fail = 0;
  for (int e = tid; e < NB * NB; e += 256) {
    const int i = e / NB, j = e % NB;
    double v = 0.0;
    if (i < nb && j <= i) v = A[(int64_t)(k + i) * C + (k + j)];
    L[i][j] = v;
    T[i][j] = 0.0;
  }
  __syncthreads();
  for (int j = 0; j < nb; ++j) {
    if (tid == 0) {
      const double d = L[j][j];
      if (!(d > 0.0) || !rq_isfinite(d)) fail = 1;
      else L[j][j] = sqrt(d);
    }
    __syncthreads();
    if (fail) break;
    const double djj = L[j][j];
    for (int i = j + 1 + tid; i < nb; i += 256) L[i][j] = L[i][j] / djj;
    __syncthreads();
    // trailing update of the lower triangle: L[i][l] -= L[i][j] * L[l][j], j < l <= i
    const int m = nb - j - 1;
    for (int e = tid; e < m * m; e += 256) {
      const int i = j + 1 + e / m, l = j + 1 + e % m;
      if (l <= i) L[i][l] = L[i][l] - L[i][j] * L[l][j];
    }
    __syncthreads();
  }
  if (fail) {
    if (tid == 0) atomicExch(info, 1);
    return;
  }
  // T = L^-1, column c by thread c: forward substitution.
  if (tid < nb) {
    const int c = tid;
    T[c][c] = 1.0 / L[c][c];
    for (int i = c + 1; i < nb; ++i) {
      double s = 0.0;
      for (int m2 = c; m2 < i; ++m2) s += L[i][m2] * T[m2][c];
      T[i][c] = -s / L[i][i];
    }
  }
  __syncthreads();
  for (int e = tid; e < nb * nb; e += 256) {
    const int i = e / nb, j = e % nb;
    const double v = T[i][j];
    Tbuf[i * NB + j] = v;
    Linv[(int64_t)(k + i) * C + (k + j)] = v;
  }
}

// Hinv[i][j] = fl32(Linv[C-1-i][C-1-j]) for j >= i, 0 below; non-finite -> info.
__global__ __launch_bounds__(256) void k_output_upper(const double* __restrict__ Linv, int C,
                                                      float* __restrict__ Hinv, int* info) {
  if (*info) return;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= C) return;
  int bad = 0;
  for (int i = blockIdx.y; i < C; i += gridDim.y) {
    float v = 0.0f;
    if (j >= i) v = (float)Linv[(int64_t)(C - 1 - i) * C + (C - 1 - j)];
    bad |= !rq_isfinite(v);
    Hinv[(int64_t)i * C + j] = v;
  }
  if (bad) atomicExch(info, 2);
}

// Hinv_init[i][j] = fl32(M[C-1-i][C-1-j]) with M = Linv^T Linv held in its lower triangle.
__global__ __launch_bounds__(256) void k_output_full(const double* __restrict__ M, int C,
                                                     float* __restrict__ Hinv_init, int* info) {
  if (*info) return;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= C) return;
  int bad = 0;
  for (int i = blockIdx.y; i < C; i += gridDim.y) {
    int a = C - 1 - i, b = C - 1 - j;
    if (b > a) { const int t = a; a = b; b = t; }
    const float v = (float)M[(int64_t)a * C + b];
    bad |= !rq_isfinite(v);
    Hinv_init[(int64_t)i * C + j] = v;
  }
  if (bad) atomicExch(info, 3);
}

// compute_safe_beta_from_reference_loss row statistics (gptq_plus_utils.py:183-193).
// One wavefront per row.
__global__ __launch_bounds__(256) void k_safe_beta(const float* __restrict__ G, int64_t ldg,
                                                   const float* __restrict__ GH0,
                                                   const float* __restrict__ Hinit, int R, int C,
                                                   float target, float* __restrict__ beta) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  float s1 = 0.0f, s2 = 0.0f;
  for (int j = lane; j < C; j += 64) {
    const float gh = GH0[(int64_t)r * C + j];
    s1 += G[(int64_t)r * ldg + j] * gh;
    s2 += (gh * gh) / Hinit[(int64_t)j * C + j];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    s1 += __shfl_xor(s1, o, 64);
    s2 += __shfl_xor(s2, o, 64);
  }
  if (lane == 0) {
    float c = s1 - s2 / (float)C;
    c = (c < target) ? target : c;                        // clamp(c, min=target)
    float ratio = (c > 0.0f) ? target / c : 0.0f;         // where(c > 0, target / c, 0)
    ratio = (ratio < 0.0f) ? 0.0f : ratio;
    ratio = (ratio > 1.0f) ? 1.0f : ratio;
    float om = 1.0f - ratio;
    om = (om < 0.0f) ? 0.0f : om;
    float b = 1.0f - sqrtf(om);
    if (b != b) b = 0.0f;                                 // nan_to_num(nan=0, posinf=1, neginf=0)
    else if (b == __builtin_inff()) b = 1.0f;
    else if (b == -__builtin_inff()) b = 0.0f;
    beta[r] = b;
  }
}

}  // namespace

extern "C" int64_t rq_chol_workspace_bytes(int C) {
  if (C <= 0) return -1;
  return (int64_t)2 * C * C * (int64_t)sizeof(double) + (int64_t)NB * NB * sizeof(double);
}

extern "C" int rq_chol_hinv_attempt(float* H_work, int C, double damp_percent, void* workspace,
                                    float* Hinv, float* Hinv_init, int* info, void* stream) {
  using namespace rq;
  if (!H_work || !workspace || !Hinv || !info || C <= 0 || !(damp_percent > 0)) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  double* A = reinterpret_cast<double*>(workspace);
  double* Linv = A + (int64_t)C * C;
  double* Tbuf = Linv + (int64_t)C * C;
  const dim3 blk(256);
  const dim3 gcol((C + 255) / 256, C < 1024 ? C : 1024);

  hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(1), 0, s, info, 0);
  hipLaunchKernelGGL(k_damp, dim3(1), blk, 0, s, H_work, C, (float)damp_percent);
  hipLaunchKernelGGL(k_reverse_to_f64, gcol, blk, 0, s, H_work, C, A, Linv);
  RQ_CHECK_LAUNCH();

  for (int k = 0; k < C; k += NB) {
    const int nb = (C - k < NB) ? (C - k) : NB;
    const int rest = C - k - nb;
    hipLaunchKernelGGL(k_chol_diag, dim3(1), blk, 0, s, A, C, k, nb, Tbuf, Linv, info);
    RQ_CHECK_LAUNCH();
    int rc;
    if (rest > 0) {
      // L_ik = A_ik T^T  (in place, rows below the panel)
      GemmArgs<double> g = gemm_args<double>(A + (int64_t)(k + nb) * C + k, C, Tbuf, NB,
                                             A + (int64_t)(k + nb) * C + k, C, rest, nb, nb, 1.0,
                                             EPI_STORE);
      g.abort_flag = info;
      if ((rc = launch_gemm(g, false, true, s))) return rc;
    }
    if (k > 0) {
      // X_k[:, 0:k] = T B_k[:, 0:k]  (in place, row block k of L^-1)
      GemmArgs<double> g = gemm_args<double>(Tbuf, NB, Linv + (int64_t)k * C, C,
                                             Linv + (int64_t)k * C, C, nb, k, nb, 1.0, EPI_STORE);
      g.abort_flag = info;
      if ((rc = launch_gemm(g, false, false, s))) return rc;
    }
    if (rest > 0) {
      // B_i[:, 0:k+nb] -= L_ik X_k
      GemmArgs<double> g = gemm_args<double>(A + (int64_t)(k + nb) * C + k, C, Linv + (int64_t)k * C,
                                             C, Linv + (int64_t)(k + nb) * C, C, rest, k + nb, nb,
                                             -1.0, EPI_ACCUM);
      g.abort_flag = info;
      if ((rc = launch_gemm(g, false, false, s))) return rc;
      // A_ij -= L_ik L_jk^T on the lower tiles of the trailing matrix
      GemmArgs<double> h = gemm_args<double>(A + (int64_t)(k + nb) * C + k, C,
                                             A + (int64_t)(k + nb) * C + k, C,
                                             A + (int64_t)(k + nb) * C + (k + nb), C, rest, rest, nb,
                                             -1.0, EPI_ACCUM);
      h.lower_only = 1;
      h.abort_flag = info;
      if ((rc = launch_gemm(h, false, true, s))) return rc;
    }
  }
  hipLaunchKernelGGL(k_output_upper, gcol, blk, 0, s, Linv, C, Hinv, info);
  RQ_CHECK_LAUNCH();
  if (Hinv_init) {
    // M = Linv^T Linv (lower tiles) into A, then Hinv_init = P M P.
    GemmArgs<double> g = gemm_args<double>(Linv, C, Linv, C, A, C, C, C, C, 1.0, EPI_STORE);
    g.krange = KR_AB_LOWER;
    g.lower_only = 1;
    g.abort_flag = info;
    int rc = launch_gemm(g, true, false, s);
    if (rc) return rc;
    hipLaunchKernelGGL(k_output_full, gcol, blk, 0, s, A, C, Hinv_init, info);
    RQ_CHECK_LAUNCH();
  }
  return RQ_OK;
}

extern "C" int rq_gptqplus_terms(const float* G_sub, int64_t ldg, const float* Hinv_init,
                                 const float* Hinv, int R_s, int C, double alpha_eff,
                                 double reference_loss, int beta_mode, float* beta, float* Z,
                                 float* GHinv, int64_t ldz, float* GH0, int* z_nonzero,
                                 void* stream) {
  using namespace rq;
  if (!G_sub || !Hinv || !beta || !Z || !GHinv || !z_nonzero || R_s <= 0 || C <= 0 || ldg < C ||
      ldz < C)
    return RQ_EINVAL;
  if (beta_mode == 1 && (!Hinv_init || !GH0)) return RQ_EINVAL;
  if (beta_mode != 0 && beta_mode != 1) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int rc;
  if (beta_mode == 1) {
    if (reference_loss <= 0) {
      // beta = zeros(R_s) (:181-183): the GEMMs below then produce exact zeros.
      hipLaunchKernelGGL(k_fill_f32, dim3(1), dim3(1), 0, s, beta, 0.0f);
      beta_mode = 0;
    } else {
      GemmArgs<float> g = gemm_args<float>(G_sub, ldg, Hinv_init, C, GH0, C, R_s, C, C, 1.0f, EPI_STORE);
      if ((rc = launch_gemm(g, false, false, s))) return rc;
      const float target = (float)(2.0 * alpha_eff * reference_loss);
      hipLaunchKernelGGL(k_safe_beta, dim3((R_s + 3) / 4), dim3(256), 0, s, G_sub, ldg, GH0,
                         Hinv_init, R_s, C, target, beta);
      RQ_CHECK_LAUNCH();
    }
  } else {
    hipLaunchKernelGGL(k_fill_f32, dim3(1), dim3(1), 0, s, beta, 0.0f);
  }
  hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(1), 0, s, z_nonzero, 0);
  RQ_CHECK_LAUNCH();
  // Z = (G_sub Hinv^T) * beta ; Hinv upper => B(k, j) = Hinv[j][k] vanishes for k < j
  GemmArgs<float> z = gemm_args<float>(G_sub, ldg, Hinv, C, Z, ldz, R_s, C, C, 1.0f, EPI_STORE);
  z.krange = KR_B_LOWER;
  z.row_scale = beta;
  z.row_bcast = (beta_mode == 0);
  z.nz_flag = z_nonzero;
  if ((rc = launch_gemm(z, false, true, s))) return rc;
  // GHinv = Z Hinv ; B(k, j) = Hinv[k][j] vanishes for k > j; all-zero Z -> zeros
  GemmArgs<float> h = gemm_args<float>(Z, ldz, Hinv, C, GHinv, ldz, R_s, C, C, 1.0f, EPI_STORE);
  h.krange = KR_B_UPPER;
  h.skip_if_zero = z_nonzero;
  if ((rc = launch_gemm(h, false, false, s))) return rc;
  return RQ_OK;
}
