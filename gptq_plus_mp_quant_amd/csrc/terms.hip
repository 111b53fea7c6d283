// GPTQ+ first-order terms of all subgroups of a layer in one call:
// GPTQPlus._compute_gradient_terms (gptq_utils/gptq_plus_utils.py:563-578) with
// compute_safe_beta_from_reference_loss (:174-194):
//   ghinv_init = G Hinv_init,  beta = f(G, ghinv_init, diag(Hinv_init)),
//   Z = (G Hinv^T) * beta,  GHinv = Z Hinv,
// per subgroup s (rows s*R_s .. of G / Z / GHinv, its own upper factor Hinv[s], U^T U = Hinv_init).
//
// beta_mode 1 never forms Hinv_init: with Y = G U^T, ghinv_init = Y U (two triangular products
// in place of a full one) and diag(Hinv_init) comes from the Cholesky chain.  The three
// products Y = G U^T, Y U and Z U are NT GEMMs (both operands k-contiguous; U^T is written
// once for the last two) on a 128x128-tile fp32 MFMA kernel, all subgroups in one launch with
// the longest K ranges first (the triangle makes tile work range from 128 to C).
#include "gemm_tile.h"

namespace {

__global__ void k_fill_f32(float* p, float v) { *p = v; }
__global__ void k_zero_i32(int* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Z[r][j] = Y[r][j] * beta[r] in place (fl32 of the fp32 product, as the reference's
// `(G @ Hinv.T) * beta_view`); nz[r / R_s] = 1 when any result of row r is non-zero or NaN.
__global__ __launch_bounds__(256) void k_row_scale_flag(float* __restrict__ Z, int64_t ldz, int R, int C,
                                                        int R_s, const float* __restrict__ beta,
                                                        int* __restrict__ nz) {
  for (int r = blockIdx.y; r < R; r += gridDim.y) {
    const float bv = beta[r];
    int any = 0;
    for (int j = blockIdx.x * 256 + threadIdx.x; j < C; j += gridDim.x * 256) {
      float* z = Z + (int64_t)r * ldz + j;
      const float v = *z * bv;
      *z = v;
      any |= (v != 0.0f) | (v != v);
    }
    // one atomic per wave only while the flag is still clear (its L2 copy is read first):
    // nearly every row is non-zero, and atomics of all waves on the few flag words serialise
    if (__any(any) && (threadIdx.x & 63) == 0 &&
        __hip_atomic_load(nz + r / R_s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0)
      atomicOr(nz + r / R_s, 1);
  }
}

// out[b] = max(out[b], max_i |x_b[i]|) as fp32 bit patterns (non-negative floats order like
// their bits, and a NaN's bits exceed +inf's) for the n values of x_b = x + b * n (grid.y = b);
// out starts at 0.  16-byte loads where x is 16-byte aligned; one atomic per workgroup.
__global__ __launch_bounds__(256) void k_absmax_bits(const float* __restrict__ x, int64_t n,
                                                     unsigned* __restrict__ out) {
  __shared__ unsigned wm[4];
  x += (int64_t)blockIdx.y * n;
  unsigned m = 0u;
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x;
  int64_t done = 0;
  if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    const int64_t n4 = n / 4;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    auto fold = [&](const float4 v) __attribute__((always_inline)) {
      m = max(m, max(max(__float_as_uint(fabsf(v.x)), __float_as_uint(fabsf(v.y))),
                     max(__float_as_uint(fabsf(v.z)), __float_as_uint(fabsf(v.w)))));
    };
    int64_t i = i0;
    for (; i + 3 * stride < n4; i += 4 * stride) {   // 4 loads in flight per thread
      const float4 v0 = x4[i], v1 = x4[i + stride], v2 = x4[i + 2 * stride], v3 = x4[i + 3 * stride];
      fold(v0);
      fold(v1);
      fold(v2);
      fold(v3);
    }
    for (; i < n4; i += stride) fold(x4[i]);
    done = 4 * n4;
  }
  for (int64_t i = done + i0; i < n; i += stride) m = max(m, __float_as_uint(fabsf(x[i])));
  for (int o = 32; o > 0; o >>= 1) m = max(m, (unsigned)__shfl_xor((int)m, o, 64));
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    m = max(max(wm[0], wm[1]), max(wm[2], wm[3]));
    if (m) atomicMax(out + blockIdx.y, m);
  }
}

// need[r / R_s] |= !(sum_k |G[r][k]| * mh[r / R_s] < 3e38) (fp64 sums; a non-finite G or mh
// fails the test).  One wavefront per row.
__global__ __launch_bounds__(256) void k_z_rows_need(const float* __restrict__ G, int64_t ldg, int R,
                                                     int C, int R_s, const float* __restrict__ mh,
                                                     int* __restrict__ need) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= R) return;
  double s = 0.0;
  for (int k = lane; k < C; k += 64) s += (double)fabsf(G[(int64_t)r * ldg + k]);
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if (lane == 0 && !(s * (double)mh[r / R_s] < 3.0e38)) atomicOr(need + r / R_s, 1);
}

// compute_safe_beta_from_reference_loss row statistics (gptq_plus_utils.py:183-193); row r
// uses its subgroup's diag(Hinv_init), hdiag + (r / R_s) * C.  One wavefront per row.
__global__ __launch_bounds__(256) void k_safe_beta(const float* __restrict__ G, int64_t ldg,
                                                   const float* __restrict__ GH0,
                                                   const float* __restrict__ hdiag, int R, int C, int R_s,
                                                   float target, float* __restrict__ beta) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  const float* hd = hdiag + (int64_t)(r / R_s) * C;
  float s1 = 0.0f, s2 = 0.0f;
  for (int j = lane; j < C; j += 64) {
    const float gh = GH0[(int64_t)r * C + j];
    s1 += G[(int64_t)r * ldg + j] * gh;
    s2 += (gh * gh) / hd[j];
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

// out[b] = in[b]^T for nb C x C matrices (32 x 32 tiles through LDS; grid.z = b).  Tiles of
// `in` strictly below the diagonal are known zero (`in` is upper triangular): their images are
// written as zeros without reading them.
__global__ __launch_bounds__(256) void k_transpose_upper(const float* __restrict__ in, float* __restrict__ out,
                                                         int C) {
  __shared__ float t[32][33];
  const int64_t off = (int64_t)blockIdx.z * C * C;
  const int bi = blockIdx.y, bj = blockIdx.x;   // source tile (rows 32 bi, columns 32 bj)
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;   // 32 x 8
  const bool zero = bi > bj;
  if (!zero) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = 32 * bi + ty + 8 * k, j = 32 * bj + tx;
      t[ty + 8 * k][tx] = (i < C && j < C) ? in[off + (int64_t)i * C + j] : 0.0f;
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int j = 32 * bj + ty + 8 * k, i = 32 * bi + tx;   // out[j][i] = in[i][j]
    if (i < C && j < C) out[off + (int64_t)j * C + i] = zero ? 0.0f : t[tx][ty + 8 * k];
  }
}

// -------------------------------------------------------------------------------------------
// NT GEMM  Cm_b[i][j] = sum_{k in range(tile)} A_b[i][k] B_b[j][k]   (b < nb, fp32)
// with the k range of a tile fixed by B's triangle: upper == 0 (B(j, k) = 0 for k < j):
// [j0, K); upper == 1 (B(j, k) = 0 for k > j): [0, min(K, j0 + 128)).
// 128 x 128 output tiles, 4 waves of 64 x 64 (2 x 2 blocks of v_mfma_f32_32x32x2f32; two
// workgroups per CU).  K advances 16 at a time through a ring of NT_STAGES LDS stages filled
// by direct global -> LDS loads issued NT_STAGES-1 steps ahead; one barrier per step.
//  - Staging: a chunk is 16 rows x 16 k (1 KB); lane L fetches row L/4, 16-byte piece
//    q = (L%4) ^ swz(row) into slot L, swz(r) = ((r >> 1) ^ (r >> 2)) & 3, so that the 16-byte
//    reads below are free of bank conflicts for every 8 or 16 consecutive rows.
//  - MFMA k order: lane half h (lane / 32) supplies k = 8h + s in sub-step s (0..7) on both
//    operands, so a lane reads its k values of a row as two 16-byte pieces (2h, 2h+1).
// Requires K % 16 == 0 and 16-byte aligned rows; edge rows read clamped (in-bounds) addresses
// and their results are not stored.
constexpr int NT_T = 128;
constexpr int NT_KS = 16;
constexpr int NT_STAGES = 4;
constexpr int NT_THREADS = 256;
constexpr int NT_CHUNK = 1024;
constexpr int NT_OPB = 8 * NT_CHUNK;          // one operand's 128 rows
constexpr int NT_STAGE = 2 * NT_OPB;

struct NtArgs {
  const float* A;
  int64_t lda, sa;     // A_b[i][k] = A[b * sa + i * lda + k]
  const float* B;
  int64_t ldb, sb;     // B_b[j][k] = B[b * sb + j * ldb + k]
  float* Cm;
  int64_t ldc, sc;
  int M, N, K;
  int upper;
  const int* skip;     // optional: skip[b] == 0 -> Cm_b = 0 (no products)
  int ntr, ntc, nb;
};

__device__ __forceinline__ int nt_swz(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }

__device__ __forceinline__ void nt_dma16(const void* g, uint8_t* l) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)l, 16, 0, 0);
}

#define NT_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

struct NtStages {
  uint8_t* s[NT_STAGES];
};

struct NtTile {
  const float* srcA[2];
  const float* srcB[2];
  int wave, lane, wr, wc, h, r;
  floatx16 acc[2][2];

  // 4 staging loads per wave and step: chunks 2 wave and 2 wave + 1 of A and of B
  __device__ __forceinline__ void stage(uint8_t* st, int kt) {
    const int64_t ko = (int64_t)kt * NT_KS;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      nt_dma16(srcA[c] + ko, st + (2 * wave + c) * NT_CHUNK);
      nt_dma16(srcB[c] + ko, st + NT_OPB + (2 * wave + c) * NT_CHUNK);
    }
  }

  // the 8 k values (8h .. 8h+7) of row `row` (0..127) of an operand region
  __device__ __forceinline__ void read_row(const uint8_t* base, int row, float (&v)[8]) const {
    const int rr = row & 15;
    const uint8_t* ch = base + (row >> 4) * NT_CHUNK + 64 * rr;
    const float4 p0 = *reinterpret_cast<const float4*>(ch + 16 * ((2 * h) ^ nt_swz(rr)));
    const float4 p1 = *reinterpret_cast<const float4*>(ch + 16 * ((2 * h + 1) ^ nt_swz(rr)));
    v[0] = p0.x; v[1] = p0.y; v[2] = p0.z; v[3] = p0.w;
    v[4] = p1.x; v[5] = p1.y; v[6] = p1.z; v[7] = p1.w;
  }

  // Step kt: wait for this wave's staging of kt (the NT_STAGES-2 later steps may still be in
  // flight), meet the other waves (their parts of kt are then in LDS, and every read of the
  // FILL stage, done in step kt-1, is over), refill FILL with step kt+NT_STAGES-1, multiply kt.
  template <int CUR, int FILL>
  __device__ __forceinline__ void step(const NtStages& L, int kt, int nk) {
    NT_WAIT_VM(4 * (NT_STAGES - 2));
    RQ_STAGE_BARRIER();
    stage(L.s[FILL], min(kt + NT_STAGES - 1, nk - 1));
    const uint8_t* st = L.s[CUR];
    float a[2][8], b[2][8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      read_row(st, 64 * wr + 32 * q + r, a[q]);
      read_row(st + NT_OPB, 64 * wc + 32 * q + r, b[q]);
    }
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int qa = 0; qa < 2; ++qa)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
          acc[qa][qb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[qa][s], b[qb][s], acc[qa][qb], 0, 0, 0);
  }
};

__global__ __launch_bounds__(NT_THREADS, 2) void k_gemm_nt128(NtArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds0[NT_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds1[NT_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds2[NT_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds3[NT_STAGE];
  static_assert(NT_STAGES == 4, "stage arrays");
  const NtStages L{{lds0, lds1, lds2, lds3}};
  // longest k ranges first: column tiles in order of falling range, each with all of its
  // (batch entry, row tile) pairs
  const int u = blockIdx.x;
  const int per = p.nb * p.ntr;
  const int cidx = u / per, rem = u % per;
  const int tj = p.upper ? p.ntc - 1 - cidx : cidx;
  const int bz = rem / p.ntr, ti = rem % p.ntr;
  const int i0 = ti * NT_T, j0 = tj * NT_T;
  float* Cb = p.Cm + bz * p.sc;
  const int tid = threadIdx.x;

  NtTile t;
  t.lane = tid & 63;
  t.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  t.wr = t.wave >> 1;
  t.wc = t.wave & 1;
  t.h = t.lane >> 5;
  t.r = t.lane & 31;
  const int k_lo = p.upper ? 0 : j0;
  const int k_hi = p.upper ? min(p.K, j0 + NT_T) : p.K;
  const int nk = (k_hi - k_lo) / NT_KS;
  const bool live = nk > 0 && !(p.skip && p.skip[bz] == 0);
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) t.acc[a][b][e] = 0.0f;

  if (live) {
    // staging sources of this wave: chunks 2 wave, 2 wave + 1 (rows 16 c + L/4)
    const int cr = t.lane >> 2;
    const int q = (t.lane & 3) ^ nt_swz(cr);
    const float* Ab = p.A + bz * p.sa;
    const float* Bb = p.B + bz * p.sb;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int row = 16 * (2 * t.wave + c) + cr;
      t.srcA[c] = Ab + (int64_t)min(i0 + row, p.M - 1) * p.lda + k_lo + 4 * q;
      t.srcB[c] = Bb + (int64_t)min(j0 + row, p.N - 1) * p.ldb + k_lo + 4 * q;
    }
#pragma unroll
    for (int s = 0; s < NT_STAGES - 1; ++s) t.stage(L.s[s], min(s, nk - 1));
    int kt = 0;
    for (; kt + 4 <= nk; kt += 4) {
      t.step<0, 3>(L, kt, nk);
      t.step<1, 0>(L, kt + 1, nk);
      t.step<2, 1>(L, kt + 2, nk);
      t.step<3, 2>(L, kt + 3, nk);
    }
    const int rest = nk - kt;
    if (rest > 0) t.step<0, 3>(L, kt, nk);
    if (rest > 1) t.step<1, 0>(L, kt + 1, nk);
    if (rest > 2) t.step<2, 1>(L, kt + 2, nk);
    NT_WAIT_VM(0);   // no staging in flight when the workgroup ends
  }
  // 32x32 block layout: column lane % 32, row 8 (e / 4) + 4 (lane / 32) + e % 4
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int j = j0 + 64 * t.wc + 32 * b + t.r;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = i0 + 64 * t.wr + 32 * a + 8 * (e >> 2) + 4 * t.h + (e & 3);
        if (i < p.M && j < p.N) Cb[(int64_t)i * p.ldc + j] = t.acc[a][b][e];
      }
    }
}

// An operand k_gemm_nt128 can stage: 16-byte aligned rows and batch strides.
bool nt_ok(const void* ptr, int64_t ld, int64_t stride) {
  return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0 && ld % 4 == 0 && stride % 4 == 0;
}

// One k_gemm_nt128 launch over nb batch entries (the caller checked K % NT_KS == 0 and nt_ok
// of A and B).
int launch_nt128(const float* A, int64_t lda, int64_t sa, const float* B, int64_t ldb, int64_t sb,
                 float* Cm, int64_t ldc, int64_t sc, int M, int N, int K, int upper, const int* skip,
                 int nb, hipStream_t s) {
  NtArgs p;
  p.A = A; p.lda = lda; p.sa = sa;
  p.B = B; p.ldb = ldb; p.sb = sb;
  p.Cm = Cm; p.ldc = ldc; p.sc = sc;
  p.M = M; p.N = N; p.K = K;
  p.upper = upper;
  p.skip = skip;
  p.ntr = (M + NT_T - 1) / NT_T;
  p.ntc = (N + NT_T - 1) / NT_T;
  p.nb = nb;
  const int64_t total = (int64_t)p.ntr * p.ntc * nb;
  if (total > 0x7fffffff) return RQ_EINVAL;
  hipLaunchKernelGGL(k_gemm_nt128, dim3((unsigned)total), dim3(NT_THREADS), 0, s, p);
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}

}  // namespace

extern "C" int rq_gptqplus_terms(const float* G, int64_t ldg, const float* hinv_diag, const float* Hinv,
                                 float* HinvT, int R_s, int nsub, int C, double alpha_eff,
                                 double reference_loss, int beta_mode, float* beta, float* Z,
                                 float* GHinv, int64_t ldz, float* GH0, int* z_nonzero, void* stream) {
  using namespace rq;
  if (!G || !Hinv || !beta || !Z || !GHinv || !z_nonzero || R_s <= 0 || nsub <= 0 || C <= 0 ||
      ldg < C || ldz < C)
    return RQ_EINVAL;
  if (beta_mode != 0 && beta_mode != 1) return RQ_EINVAL;
  if (beta_mode == 1 && reference_loss > 0 && (!hinv_diag || !GH0)) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int R = R_s * nsub;
  const int64_t CC = (int64_t)C * C;
  const int rows_grid = R < 65535 ? R : 65535;
  const int cols_grid = (C + 255) / 256 < 8 ? (C + 255) / 256 : 8;
  int rc;
  hipLaunchKernelGGL(k_zero_i32, dim3((nsub + 255) / 256), dim3(256), 0, s, z_nonzero, nsub);
  RQ_CHECK_LAUNCH();
  if (beta_mode == 1 && reference_loss > 0) {
    // Y = G Hinv^T (the reference's G Hinv^T before its beta scaling) into Z; Hinv^T; then
    // ghinv_init = Y Hinv = G Hinv^T Hinv = G Hinv_init (:180) into GH0.
    const bool fast = HinvT && C % NT_KS == 0 && nt_ok(G, ldg, (int64_t)R_s * ldg) && nt_ok(Hinv, C, CC) &&
                      nt_ok(HinvT, C, CC) && nt_ok(Z, ldz, (int64_t)R_s * ldz);
    if (fast) {
      if ((rc = launch_nt128(G, ldg, (int64_t)R_s * ldg, Hinv, C, CC, Z, ldz, (int64_t)R_s * ldz, R_s, C, C, 0,
                             nullptr, nsub, s)))
        return rc;
      hipLaunchKernelGGL(k_transpose_upper, dim3((C + 31) / 32, (C + 31) / 32, nsub), dim3(256), 0, s, Hinv,
                         HinvT, C);
      RQ_CHECK_LAUNCH();
      if ((rc = launch_nt128(Z, ldz, (int64_t)R_s * ldz, HinvT, C, CC, GH0, C, (int64_t)R_s * C, R_s, C, C, 1,
                             nullptr, nsub, s)))
        return rc;
    } else {
      for (int b = 0; b < nsub; ++b) {
        GemmArgs<float> y = gemm_args<float>(G + (int64_t)b * R_s * ldg, ldg, Hinv + b * CC, C,
                                             Z + (int64_t)b * R_s * ldz, ldz, R_s, C, C, 1.0f, EPI_STORE);
        y.krange = KR_B_LOWER;
        if ((rc = launch_gemm(y, false, true, s))) return rc;
        GemmArgs<float> g = gemm_args<float>(Z + (int64_t)b * R_s * ldz, ldz, Hinv + b * CC, C,
                                             GH0 + (int64_t)b * R_s * C, C, R_s, C, C, 1.0f, EPI_STORE);
        g.krange = KR_B_UPPER;
        if ((rc = launch_gemm(g, false, false, s))) return rc;
      }
    }
    const float target = (float)(2.0 * alpha_eff * reference_loss);
    hipLaunchKernelGGL(k_safe_beta, dim3((R + 3) / 4), dim3(256), 0, s, G, ldg, GH0, hinv_diag, R, C, R_s,
                       target, beta);
    // Z = Y * beta (row-wise, in place), then GHinv = Z Hinv
    hipLaunchKernelGGL(k_row_scale_flag, dim3(cols_grid, rows_grid), dim3(256), 0, s, Z, ldz, R, C, R_s,
                       (const float*)beta, z_nonzero);
    RQ_CHECK_LAUNCH();
    if (fast)
      return launch_nt128(Z, ldz, (int64_t)R_s * ldz, HinvT, C, CC, GHinv, ldz, (int64_t)R_s * ldz, R_s, C, C, 1,
                          z_nonzero, nsub, s);
    for (int b = 0; b < nsub; ++b) {
      GemmArgs<float> h = gemm_args<float>(Z + (int64_t)b * R_s * ldz, ldz, Hinv + b * CC, C,
                                           GHinv + (int64_t)b * R_s * ldz, ldz, R_s, C, C, 1.0f, EPI_STORE);
      h.krange = KR_B_UPPER;
      h.skip_if_zero = z_nonzero + b;
      if ((rc = launch_gemm(h, false, false, s))) return rc;
    }
    return RQ_OK;
  }
  // beta = 0: zeros(R_s) for beta_mode 1 with reference_loss <= 0 (:181-183), a scalar 0
  // otherwise (:575).  Z = (G Hinv^T) * 0 is zero unless a product or a partial sum of
  // G Hinv^T is not finite (then the reference's 0 * inf is NaN).  Every partial sum of row r
  // is bounded by sum_k |G[r][k]| * max|Hinv|, so when that bound stays well inside the fp32
  // range for every row of a subgroup (and G is finite), its Z is zero and the products are
  // skipped (z_nonzero stays 0; only zeros are stored).  Otherwise z_nonzero is raised and Z
  // is formed.  max|Hinv| of subgroup b passes through GHinv[b] (as bits; GHinv is written
  // afterwards).
  hipLaunchKernelGGL(k_fill_f32, dim3(1), dim3(1), 0, s, beta, 0.0f);
  unsigned* mh = reinterpret_cast<unsigned*>(GHinv);
  hipLaunchKernelGGL(k_zero_i32, dim3((nsub + 255) / 256), dim3(256), 0, s, reinterpret_cast<int*>(mh), nsub);
  hipLaunchKernelGGL(k_absmax_bits, dim3(C >= 2048 ? 256 : 64, nsub), dim3(256), 0, s, Hinv, CC, mh);
  hipLaunchKernelGGL(k_z_rows_need, dim3((R + 3) / 4), dim3(256), 0, s, G, ldg, R, C, R_s,
                     (const float*)mh, z_nonzero);
  RQ_CHECK_LAUNCH();
  for (int b = 0; b < nsub; ++b) {
    // Z = (G Hinv^T) * 0 ; Hinv upper => B(k, j) = Hinv[j][k] vanishes for k < j
    GemmArgs<float> z = gemm_args<float>(G + (int64_t)b * R_s * ldg, ldg, Hinv + b * CC, C,
                                         Z + (int64_t)b * R_s * ldz, ldz, R_s, C, C, 1.0f, EPI_STORE);
    z.krange = KR_B_LOWER;
    z.row_scale = beta;
    z.row_bcast = 1;
    z.skip_if_zero = z_nonzero + b;
    if ((rc = launch_gemm(z, false, true, s))) return rc;
  }
  for (int b = 0; b < nsub; ++b) {
    // GHinv = Z Hinv ; B(k, j) = Hinv[k][j] vanishes for k > j; all-zero Z -> zeros
    GemmArgs<float> h = gemm_args<float>(Z + (int64_t)b * R_s * ldz, ldz, Hinv + b * CC, C,
                                         GHinv + (int64_t)b * R_s * ldz, ldz, R_s, C, C, 1.0f, EPI_STORE);
    h.krange = KR_B_UPPER;
    h.skip_if_zero = z_nonzero + b;
    if ((rc = launch_gemm(h, false, false, s))) return rc;
  }
  return RQ_OK;
}
