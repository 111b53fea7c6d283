// Damped Cholesky chain (GPTQPlus._compute_hessian_inverse_with_fallback,
// gptq_utils/gptq_plus_utils.py:494-561).
//
// The reference computes chol(H) -> cholesky_inverse -> chol(H^-1, upper) in fp32.  Here the
// upper factor U of H^-1 (U^T U = H^-1) is obtained with ONE factorisation: with P the
// index-reversal permutation and L L^T = P H P,  U = P L^-1 P.  The factorisation and the
// inverse L^-1 run together in one right-looking blocked pass in fp64 (64-wide blocks
// inside 256-wide panels; from C = 8192 512-wide panels, each factored as two 256-wide
// halves):
//   per block k:  L_kk = chol(A_kk), T = L_kk^-1, L_ik = A_ik T^T and X_k = T B_k (row block k
//                 of L^-1) in one launch (k_chol_step: every workgroup factors the 64 x 64
//                 block itself, then does its GEMM tiles),
//                 A_ij -= L_ik L_jk^T (lower tiles),  B_i -= L_ik X_k   (fp64 MFMA GEMMs),
// where B accumulates I - sum_m L_im X_m.  The updates of the trailing matrix and of the rows
// of B below a panel are applied once per panel (rank 256 / 512) instead of once per block,
// by k_panel_update (128x128 tiles, direct global->LDS staging); the part of that update past
// the next panel runs on a second stream while the next panel is factored (look-ahead).  H^-1 itself (Hinv_init) is
// P (L^-T L^-1) P and is only formed when asked for; its diagonal (all that the GPTQ+ step
// size needs of it) comes from the column norms of L^-1.  A non-positive or non-finite pivot, or
// a non-finite result, raises the device `info` flag; later kernels of the same attempt exit
// early.
#include "gemm_tile.h"

#include <algorithm>

namespace {

constexpr int NB = 64;     // diagonal block (factored and inverted by one workgroup)
// Outer panel width: 256, or 512 from C = 8192 on.  The panel update re-reads and re-writes
// its output tile once per panel, so wider panels halve that epilogue's share; the extra
// in-panel work (C^2 NBW / 2 flops) stays ~1 % of the C^3 chain there.
__host__ __device__ constexpr int panel_width(int C) { return C >= 8192 ? 512 : 256; }


constexpr int MAXBATCH = 64;
struct BatchCfg {
  float damp[MAXBATCH];
  int active[MAXBATCH];
};

__global__ void k_init_info(int* info, int nb, BatchCfg cfg) {
  const int b = threadIdx.x;
  if (b < nb) info[b] = cfg.active[b] ? 0 : -1;
}

// H_work[i,i] += fl32(p) * mean(diag(H_work)).  One workgroup per batch entry.
__global__ __launch_bounds__(256) void k_damp(float* __restrict__ H, int C, BatchCfg cfg,
                                              const int* __restrict__ info) {
  __shared__ double part[256];
  const int b = blockIdx.x;
  if (info[b]) return;
  H += (int64_t)b * C * C;
  const float p = cfg.damp[b];
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

// A = P H_work P in fp64 (full square), Linv = 0.  grid.z = batch entry.
__global__ __launch_bounds__(256) void k_reverse_to_f64(const float* __restrict__ H, int C,
                                                        double* __restrict__ A,
                                                        double* __restrict__ Linv, int64_t ws,
                                                        const int* __restrict__ info) {
  const int b = blockIdx.z;
  if (info[b]) return;
  H += (int64_t)b * C * C;
  A += b * ws;
  Linv += b * ws;
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= C) return;
  for (int i = blockIdx.y; i < C; i += gridDim.y) {
    A[(int64_t)i * C + j] = (double)H[(int64_t)(C - 1 - i) * C + (C - 1 - j)];
    Linv[(int64_t)i * C + j] = 0.0;
  }
}

// 1/sqrt(d) and sqrt(d) in fp64 from the hardware estimate (relative error 2^-24 on gfx950,
// measured over 2^20 random inputs) and one Newton step y <- y (3 - d y^2) / 2, which squares
// the error: 2^-47.8 measured, far below what the fp32 input and output resolve.
__device__ __forceinline__ void rsqrt_newton(double d, double& rs, double& sq) {
  double y = __builtin_amdgcn_rsq(d);
  const double h = 0.5 * d;
  y = y * __builtin_fma(-h * y, y, 1.5);
  rs = y;
  sq = d * y;
}

// Factor the nb x nb diagonal block of A at (k, k) and invert it; one workgroup of 4 waves per
// batch entry (rows >= nb are identity padding).  Blocked by 16, in LDS:
//   for b = 0..3:  D = A_bb:  L_bb = chol(D) and T_bb = L_bb^-1            (16 x 16, in-wave)
//                  L_ib = A_ib T_bb^T (i > b),  X_b = T_bb B_b[:, 0:16b]   (MFMA)
//                  A_ij -= L_ib L_jb^T (b < j <= i),  B_i[:, 0:16b+16] -= L_ib X_b  (i > b)
// with B = I at the start; row block b of B becomes X_b, row block b of T = L^-1 (its diagonal
// block T_bb).  The block products are 16 x 16 x 16 on v_mfma_f64_16x16x4f64, spread over the 4
// waves, two barriers per block column.
//  - The 16 x 16 factorisation runs in every wave on the same LDS data (no barrier; the waves
//    reach the same verdict on the pivots).  Lane 4r + q holds D[r][4q .. 4q+3] and the same
//    entries of the running inverse W (= I at the start).  Columns go in groups of 4: the
//    lanes of the group's rows publish those rows of D and W in a per-wave LDS buffer (one
//    wave's LDS accesses complete in order); every lane factors the 4 x 4 pivot block
//    (L_P, with 1/sqrt of each pivot), solves for the L entries of its own row and of its 4
//    columns in the group (D is symmetric, so the published rows are also the columns), forms
//    the group's rows of T, X = L_P^-1 W_group, and rows below the group subtract their rank-4
//    products from D and W.  After 4 groups W = T_bb.
constexpr int CD_THREADS = 256;
constexpr int DLS = NB + 2;                 // LDS row stride of the block and of B (doubles)
constexpr int OPS = 17;                     // row stride of a wave's T_bb operand copy

__device__ __forceinline__ doublex4 mfma_f64(double a, double b, doublex4 c) {
  return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
}

// Leaves T in Bm (lower, exact zeros above, the identity on the padding) and returns 0, or
// returns 1 when a pivot is not positive and finite (every wave of the workgroup sees the same),
// or 2 when `skip` is set (the entry's attempt has already failed).
__device__ __forceinline__ int chol_diag_lds(const double* __restrict__ A, int C, int k, int nb, int skip,
                                             double* __restrict__ Am, double* __restrict__ Bm,
                                             double (*pub)[4 * 32], double (*opnd)[16 * OPS]) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // The block, symmetric, from its lower triangle (only rows and columns < nb are read; the
  // padding is the identity), and B = I.  A wave reads two whole rows per instruction: thread
  // t, step q takes the column pair 2 (t % 32) of row (t + 256 q) / 32 (16-byte loads when the
  // rows are aligned and whole, else clamped column indices); all loads go out before the
  // LDS writes.
  {
    double2 v[8];
    const bool vec = (nb == NB) && (C & 1) == 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int e = tid + 256 * q, r = e >> 5, c = 2 * (e & 31);
      const double* rowp = A + (int64_t)(k + min(r, nb - 1)) * C + k;
      if (vec) {
        v[q] = *reinterpret_cast<const double2*>(rowp + c);
      } else {
        v[q].x = rowp[min(c, nb - 1)];
        v[q].y = rowp[min(c + 1, nb - 1)];
      }
    }
    if (skip) return 2;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int e = tid + 256 * q, r = e >> 5, c = 2 * (e & 31);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int cc = c + h;
        Bm[r * DLS + cc] = (r == cc) ? 1.0 : 0.0;
        if (cc <= r) {
          const double x = (r < nb) ? (h ? v[q].y : v[q].x) : ((r == cc) ? 1.0 : 0.0);
          Am[r * DLS + cc] = x;
          Am[cc * DLS + r] = x;
        }
      }
    }
  }
  __syncthreads();

  const int fr = lane >> 2, fq = lane & 3;      // in-wave 16 x 16 layout: row fr, columns 4 fq ..
  const int mi = lane & 15, mk = lane >> 4;     // MFMA operand: row / column mi, k mk
  double* pw = pub[wave];
  double* ow = opnd[wave];
  bool bad = false;
  for (int bb = 0; bb < 4; ++bb) {
    const int o = 16 * bb;
    // (1) L_bb and T_bb = W, in every wave
    double d[4], w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d[i] = Am[(o + fr) * DLS + o + 4 * fq + i];
      w[i] = (fr == 4 * fq + i) ? 1.0 : 0.0;
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      // columns j0 .. j0+3: the group's 4 rows of D and W are published, every lane factors
      // the 4 x 4 pivot block P, forms the L entries of its row and of its columns in the
      // group, the group's rows of T (X = L_P^-1 W_group) and applies the rank-4 updates
      const int j0 = 4 * g, own = fr - j0;
      if (own >= 0 && own < 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pw[own * 32 + 4 * fq + i] = d[i];
          pw[own * 32 + 16 + 4 * fq + i] = w[i];
        }
      }
      // lanes read what other lanes wrote: keep the compiler from moving the reads above the
      // writes (the hardware runs a wave's LDS accesses in order)
      __builtin_amdgcn_wave_barrier();
      double P[4][4], u[4][4], wv[4][4], ur[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          P[m][i] = pw[m * 32 + j0 + i];
          u[m][i] = pw[m * 32 + 4 * fq + i];
          wv[m][i] = pw[m * 32 + 16 + 4 * fq + i];
        }
        ur[m] = pw[m * 32 + fr];
      }
      __builtin_amdgcn_wave_barrier();   // the next group's writes stay after these reads
      double Lp[4][4], rs[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        double dm = P[m][m];
#pragma unroll
        for (int q = 0; q < m; ++q) dm = __builtin_fma(-Lp[m][q], Lp[m][q], dm);
        const bool ok = dm > 0.0 && rq_isfinite(dm);
        bad |= !ok;
        double r1, sq;
        rsqrt_newton(ok ? dm : 1.0, r1, sq);    // no branch: a failed pivot ends the block anyway
        rs[m] = r1;
        Lp[m][m] = sq;
#pragma unroll
        for (int m2 = m + 1; m2 < 4; ++m2) {
          double v = P[m2][m];
#pragma unroll
          for (int q = 0; q < m; ++q) v = __builtin_fma(-Lp[m2][q], Lp[m][q], v);
          Lp[m2][m] = v * rs[m];
        }
      }
      double lr[4], lc[4][4], X[4][4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        double v = ur[m];
#pragma unroll
        for (int q = 0; q < m; ++q) v = __builtin_fma(-lr[q], Lp[m][q], v);
        lr[m] = v * rs[m];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          double c = u[m][i], x = wv[m][i];
#pragma unroll
          for (int q = 0; q < m; ++q) {
            c = __builtin_fma(-lc[i][q], Lp[m][q], c);
            x = __builtin_fma(-Lp[m][q], X[q][i], x);
          }
          lc[i][m] = c * rs[m];
          X[m][i] = x * rs[m];
        }
      }
      const bool below = fr >= j0 + 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        double nd = d[i], nw = w[i];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          nd = __builtin_fma(-lr[m], lc[i][m], nd);
          nw = __builtin_fma(-lr[m], X[m][i], nw);
        }
        double wn = below ? nw : w[i];
#pragma unroll
        for (int m = 0; m < 4; ++m) wn = (own == m) ? X[m][i] : wn;
        d[i] = below ? nd : d[i];
        w[i] = wn;
      }
    }
    if (bad) break;                            // the same in every wave
    // (2) T_bb as an MFMA operand (element [mi][4 kk + mk]), this wave's copy
#pragma unroll
    for (int i = 0; i < 4; ++i) ow[fr * OPS + 4 * fq + i] = w[i];
    __builtin_amdgcn_wave_barrier();
    double top[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) top[kk] = ow[mi * OPS + 4 * kk + mk];
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) Bm[(o + fr) * DLS + o + 4 * fq + i] = w[i];
    } else {
      // three tasks per block column: L_ib = A_ib T_bb^T for i = bb+1 .. 3, then
      // X_b[:, 16m ..] = T_bb B_b[:, 16m ..] for m = 0 .. bb-1 (both in place)
      const int t = wave - 1;
      doublex4 acc = {0.0, 0.0, 0.0, 0.0};
      if (t < 3 - bb) {
        const int i0 = 16 * (bb + 1 + t);
        double av[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) av[kk] = Am[(i0 + mi) * DLS + o + 4 * kk + mk];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc = mfma_f64(av[kk], top[kk], acc);
#pragma unroll
        for (int e = 0; e < 4; ++e) Am[(i0 + mk + 4 * e) * DLS + o + mi] = acc[e];
      } else {
        const int m0 = 16 * (t - (3 - bb));
        double bv[4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) bv[kk] = Bm[(o + 4 * kk + mk) * DLS + m0 + mi];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) acc = mfma_f64(top[kk], bv[kk], acc);
#pragma unroll
        for (int e = 0; e < 4; ++e) Bm[(o + mk + 4 * e) * DLS + m0 + mi] = acc[e];
      }
    }
    __syncthreads();
    if (bb == 3) break;
    // (3) trailing blocks: A_ij (b < j <= i, the next diagonal block first), then B_i[:, m]
    const int nA = (3 - bb) * (4 - bb) / 2, nT = nA + (3 - bb) * (bb + 1);
    for (int t = wave; t < nT; t += 4) {
      int bi, bj;
      bool isA = t < nA;
      if (isA) {           // j = bb+1 .. 3, i = j .. 3, column by column
        int u = t;
        bj = bb + 1;
        while (u >= 4 - bj) {
          u -= 4 - bj;
          ++bj;
        }
        bi = bj + u;
      } else {             // i = bb+1 .. 3, m = 0 .. bb
        const int u = t - nA;
        bi = bb + 1 + u / (bb + 1);
        bj = u % (bb + 1);
      }
      double* Cm = isA ? Am : Bm;
      doublex4 acc;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = Cm[(16 * bi + mk + 4 * e) * DLS + 16 * bj + mi];
      double av[4], bv[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        av[kk] = -Am[(16 * bi + mi) * DLS + o + 4 * kk + mk];
        bv[kk] = isA ? Am[(16 * bj + mi) * DLS + o + 4 * kk + mk] : Bm[(o + 4 * kk + mk) * DLS + 16 * bj + mi];
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) acc = mfma_f64(av[kk], bv[kk], acc);
#pragma unroll
      for (int e = 0; e < 4; ++e) Cm[(16 * bi + mk + 4 * e) * DLS + 16 * bj + mi] = acc[e];
    }
    __syncthreads();
  }
  return bad ? 1 : 0;
}

// One diagonal block step of the chain, in one launch: every workgroup factors and inverts the
// 64 x 64 diagonal block at (j, j) (chol_diag_lds: the same arithmetic in each, so the same T),
// then computes its share of the 64-wide GEMM tiles that use T:
//   tiles u < n1:   L_ij = A_ij T^T   (rows j+jb+64u .. of the block column, in place)
//   tiles u >= n1:  X_j[:, 64v ..] = T B_j[:, 64v ..]   (v = u - n1: row block j of L^-1, in place)
// The tile is staged in LDS (the block's buffer, free once T is formed) and multiplied on
// v_mfma_f64_16x16x4f64, 4 waves of 32 x 32.  Workgroup 0 of each entry writes T to Linv's
// diagonal block; a failed pivot is recorded by workgroup 0 in `info`.  Redundant factoring in
// every workgroup replaces a separate launch per block: the factorisation is latency-bound and
// the GEMM tiles need only T.
constexpr int STEP_SLOTS = 512;   // workgroups of k_chol_step resident at once (2 per CU)
struct StepArgs {
  double* A;
  double* Linv;
  int C, j, jb;
  int n1, n2;       // lij tiles (rows below the block, 64 at a time), xj tiles (64 columns of 0 .. j)
  int64_t ws;
  int* info;
};

__global__ __launch_bounds__(CD_THREADS) void k_chol_step(StepArgs p) {
  __shared__ __attribute__((aligned(16))) double Am[NB * DLS];
  __shared__ __attribute__((aligned(16))) double Bm[NB * DLS];
  __shared__ __attribute__((aligned(16))) double pub[4][4 * 32];
  __shared__ __attribute__((aligned(16))) double opnd[4][16 * OPS];
  const int b = blockIdx.z;
  int* info = p.info + b;
  const int skip = *info;
  double* A = p.A + b * p.ws;
  double* Linv = p.Linv + b * p.ws;
  const int C = p.C, j = p.j, jb = p.jb;
  const int rc = chol_diag_lds(A, C, j, jb, skip, Am, Bm, pub, opnd);
  if (rc) {
    if (rc == 1 && blockIdx.x == 0 && threadIdx.x == 0) atomicExch(info, 1);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (blockIdx.x == 0) {
    // T into Linv's diagonal block, one whole row per wave and instruction
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const int e = tid + 256 * q, r = e >> 6, c = e & 63;
      if (r < jb && c < jb) Linv[(int64_t)(j + r) * C + (j + c)] = Bm[r * DLS + c];
    }
  }
  const int mi = lane & 15, mk = lane >> 4;
  const int wr = wave >> 1, wc = wave & 1;
  const int ntiles = p.n1 + p.n2;
  for (int u = blockIdx.x; u < ntiles; u += gridDim.x) {
    const bool lij = u < p.n1;
    // the tile: lij rows j+jb+64u .., columns j .. j+jb; xj rows j .. j+jb, columns 64v ..
    // (clamped in-bounds reads: a padding row or column only meets a zero of T)
    const int r0 = lij ? j + jb + 64 * u : j;
    const int c0 = lij ? j : 64 * (u - p.n1);
    const int rmax = lij ? C - 1 : j + jb - 1;
    const int cmax = lij ? j + jb - 1 : j - 1;
    __syncthreads();                  // the previous tile's reads of Am are done
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int e = tid + 256 * q, r = e >> 5, c = 2 * (e & 31);
      const double* src = (lij ? A : Linv) + (int64_t)min(r0 + r, rmax) * C;
      Am[r * DLS + c] = src[min(c0 + c, cmax)];
      Am[r * DLS + c + 1] = src[min(c0 + c + 1, cmax)];
    }
    __syncthreads();
    doublex4 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int q = 0; q < 2; ++q) acc[a][q] = doublex4{0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      const int kx = 4 * kk + mk;
      double av[2], bv[2];
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int rr = 32 * wr + 16 * a + mi, cc = 32 * wc + 16 * a + mi;
        av[a] = lij ? Am[rr * DLS + kx] : Bm[rr * DLS + kx];          // A_ij[r][k] / T[r][k]
        bv[a] = lij ? Bm[cc * DLS + kx] : Am[kx * DLS + cc];          // T[c][k] / B_j[k][c]
      }
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int q = 0; q < 2; ++q) acc[a][q] = mfma_f64(av[a], bv[q], acc[a][q]);
    }
    double* dst = lij ? A : Linv;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = r0 + 32 * wr + 16 * a + mk + 4 * e, c = c0 + 32 * wc + 16 * q + mi;
          if (r <= rmax && c <= cmax) dst[(int64_t)r * C + c] = acc[a][q][e];
        }
  }
}

// Hinv[i][j] = fl32(Linv[C-1-i][C-1-j]) for j >= i, 0 below; non-finite -> info.
__global__ __launch_bounds__(256) void k_output_upper(const double* __restrict__ Linv, int C,
                                                      float* __restrict__ Hinv, int64_t ws,
                                                      int* info_all) {
  const int b = blockIdx.z;
  int* info = info_all + b;
  if (*info) return;
  Linv += b * ws;
  Hinv += (int64_t)b * C * C;
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
                                                     float* __restrict__ Hinv_init, int64_t ws,
                                                     int* info_all) {
  const int b = blockIdx.z;
  int* info = info_all + b;
  if (*info) return;
  M += b * ws;
  Hinv_init += (int64_t)b * C * C;
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

// diag(H^-1)[i] = sum_{k >= p} Linv[k][p]^2 with p = C-1-i (the diagonal of P Linv^T Linv P),
// in two passes: fp64 partial sums over nch = gridDim.y row chunks (`part`, nch x C doubles per
// batch entry, at stride ws), then their sum in chunk order, rounded to fp32; non-finite ->
// info 3 (as k_output_full).
__host__ __device__ constexpr int diag_chunks(int C) { return C >= 256 ? 16 : 1; }   // nch * C <= C * C
__global__ __launch_bounds__(256) void k_diag_partial(const double* __restrict__ Linv, int C,
                                                      double* __restrict__ part, int64_t ws,
                                                      const int* __restrict__ info_all) {
  const int b = blockIdx.z;
  if (info_all[b]) return;
  Linv += b * ws;
  part += b * ws;
  const int p = blockIdx.x * 256 + threadIdx.x;
  if (p >= C) return;
  const int rows = (C + gridDim.y - 1) / gridDim.y;
  const int k0 = blockIdx.y * rows, k1 = min(C, k0 + rows);
  double s = 0.0;
  for (int k = max(k0, p); k < k1; ++k) {
    const double v = Linv[(int64_t)k * C + p];
    s = __builtin_fma(v, v, s);
  }
  part[(int64_t)blockIdx.y * C + p] = s;
}

__global__ __launch_bounds__(256) void k_diag_final(const double* __restrict__ part, int C, int nch, int64_t ws,
                                                    float* __restrict__ diag, int* info_all) {
  const int b = blockIdx.z;
  int* info = info_all + b;
  if (*info) return;
  part += b * ws;
  const int p = blockIdx.x * 256 + threadIdx.x;
  if (p >= C) return;
  double s = 0.0;
  for (int c = 0; c < nch; ++c) s += part[(int64_t)c * C + p];
  const float v = (float)s;
  diag[(int64_t)b * C + (C - 1 - p)] = v;
  if (!rq_isfinite(v)) atomicExch(info, 3);
}

// ---------------------------------------------------------------------------------------------
// The two rank-K updates that follow each outer panel (K = NBW = 256 or 512 columns k .. k+K of L, rows
// pe .. C), in one launch:
//   SYRK part:  A[pe:, pe:] -= Lp Lp^T       (lower 128-tiles; Lp = L[pe:, k:k+K])
//   row part:   Linv[pe:, 0:pe] -= Lp X      (X = Linv[k:k+K, 0:pe], row block of L^-1)
// 128 x 128 output tiles, 8 waves of 32 x 64 (2 x 4 blocks of v_mfma_f64_16x16x4f64; two
// workgroups per CU give 4 waves per SIMD).  K advances 8 at a time through a ring of PSTAGES
// LDS stages filled by direct global -> LDS loads (16 bytes per lane) issued PSTAGES-1 steps
// ahead; one barrier per step.
//  - Operands stored k-contiguous (Lp for both sides of the SYRK, Lp for the row part): a
//    staging chunk is 16 rows x 8 k (1 KB); lane L fetches row L/4, k pair p = (L%4) ^
//    ((row/4)%4) into LDS slot L, so the four lanes of a row read its 64 contiguous bytes and
//    the 16 rows of one k pair sit in 16 different bank groups.
//  - X (stored j-contiguous) is staged as 8 k-rows of 128 j (1 KB each, 64 B apart).
//  - MFMA k order: in sub-step s of a stage the lanes of group g (= lane / 16) supply
//    k = 2g + s on both operands, so a k-contiguous operand is one 16-byte LDS read per
//    16 x 8 block for both sub-steps.
// Edge rows / columns read clamped (in-bounds) addresses; their results are not stored.
constexpr int PT = 128;
constexpr int PKS = 8;                      // k per stage
constexpr int PSTAGES = 4;
constexpr int PCHUNK = 1024;
constexpr int PXROW = PCHUNK + 64;          // X k-row stride in a stage
constexpr int PA_BYTES = 8 * PCHUNK;
constexpr int PSTAGE = PA_BYTES + 8 * PXROW;

// SYRK part: Atr[i][j] -= sum_k Lp[i][k] Lp[j][k] for i < ms, j < ns <= ms, lower tiles
// (tj <= ti); row part: Brow[i][j] -= sum_k Lp[i][k] X[k][j] for i < mr <= ms, j < nr.
// After a panel: ms = ns = mr = C - pe, nr = pe.  Inside a panel (block j of width jb):
// ms = rows below the block, ns = mr = panel columns right of it, nr = j + jb.
struct PanelArgs {
  const double* Lp;    // Lp[i * ld + kk], column kk < K
  const double* X;     // X[kk * ld + j]
  double* Atr;
  double* Brow;
  int64_t ld;
  int K;
  int ms, ns, mr, nr;
  int ntr, ntc;        // SYRK row / column tiles
  int nsy;             // SYRK tiles (lower trapezoid)
  int nrr, nrc;        // row-part row / column tiles
  int per_batch;       // nsy + nrr * nrc
  int64_t ws;          // batch stride (doubles)
  const int* info;
  int total;           // per_batch * nb
};

__device__ __forceinline__ void lds_dma16(const void* g, uint8_t* l) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)l, 16, 0, 0);
}

// s_waitcnt with only the vector-memory counter limited (gfx9 encoding).
#define PWAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

// The ring: PSTAGES separate __shared__ arrays.  The k loop is unrolled by PSTAGES so every
// stage index is a compile-time constant: the compiler can then tell the global -> LDS loads in
// flight to other stages from the stage being read, and does not wait for them.
struct PStages {
  uint8_t* s[PSTAGES];
};

template <bool SYRK>
struct PanelTile {
  const PanelArgs& p;
  const double* srcA;
  const double* srcB;
  int wave, lane, wr, wc, g, r, slot, nk;
  bool live;
  doublex4 acc[2][4];

  __device__ __forceinline__ PanelTile(const PanelArgs& pp, int64_t boff, int i0, int j0, int ti, int tj)
      : p(pp) {
    const int tid = threadIdx.x;
    lane = tid & 63;
    wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    wr = wave >> 1;                          // rows 32 wr .. 32 wr + 31
    wc = wave & 1;                           // columns 64 wc .. 64 wc + 63
    g = lane >> 4;
    r = lane & 15;
    slot = 4 * r + (g ^ ((r >> 2) & 3));
    nk = p.K / PKS;
    live = !(SYRK && ti == tj && wr < 2 * wc);   // inside a 64-block strictly above the diagonal
    const int M = SYRK ? p.ms : p.mr, N = SYRK ? p.ns : p.nr;
    const double* Lp = p.Lp + boff;
    // this wave's staging sources: chunk `wave` of each operand
    const int cr = lane >> 2, kp = (lane & 3) ^ ((cr >> 2) & 3);
    const int c = wave;
    srcA = Lp + (int64_t)min(i0 + 16 * c + cr, M - 1) * p.ld + 2 * kp;
    if (SYRK) srcB = Lp + (int64_t)min(j0 + 16 * c + cr, N - 1) * p.ld + 2 * kp;
    else srcB = p.X + boff + (int64_t)c * p.ld + min(j0 + 2 * lane, N - 2);
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[a][b][e] = 0.0;
  }

  // 2 staging loads per wave: chunk `wave` of A and of B
  __device__ __forceinline__ void stage(uint8_t* st, int kt) {
    const int64_t ka = (int64_t)kt * PKS;
    lds_dma16(srcA + ka, st + wave * PCHUNK);
    if (SYRK) lds_dma16(srcB + ka, st + PA_BYTES + wave * PCHUNK);
    else lds_dma16(srcB + ka * p.ld, st + PA_BYTES + wave * PXROW);
  }

  // Step kt: wait for this wave's staging of kt (the PSTAGES-2 later steps may still be in
  // flight), meet the other waves (their parts of kt are then in LDS, and every read of the
  // FILL stage, done in step kt-1, is over), refill FILL with step kt+PSTAGES-1, multiply kt.
  template <int CUR, int FILL>
  __device__ __forceinline__ void step(const PStages& L, int kt) {
    PWAIT_VM(2 * (PSTAGES - 2));
    RQ_STAGE_BARRIER();
    stage(L.s[FILL], min(kt + PSTAGES - 1, nk - 1));
    if (!live) return;
    const uint8_t* st = L.s[CUR];
    double2 av[2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
      av[rb] = *reinterpret_cast<const double2*>(st + (2 * wr + rb) * PCHUNK + 16 * slot);
    double bv[2][4];
    if (SYRK) {
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const double2 v = *reinterpret_cast<const double2*>(st + PA_BYTES + (4 * wc + cb) * PCHUNK + 16 * slot);
        bv[0][cb] = v.x;
        bv[1][cb] = v.y;
      }
    } else {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
          bv[s2][cb] = *reinterpret_cast<const double*>(st + PA_BYTES + (2 * g + s2) * PXROW +
                                                        8 * (64 * wc + 16 * cb + r));
    }
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
        acc[rb][cb] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[rb].x, bv[0][cb], acc[rb][cb], 0, 0, 0);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
        acc[rb][cb] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[rb].y, bv[1][cb], acc[rb][cb], 0, 0, 0);
  }
};

template <bool SYRK>
__device__ __forceinline__ void panel_tile(const PanelArgs& p, int64_t boff, int ti, int tj, const PStages& L) {
  const int i0 = ti * PT, j0 = tj * PT;
  PanelTile<SYRK> t(p, boff, i0, j0, ti, tj);
  const int nk = t.nk;
  static_assert(PSTAGES == 4, "unrolled stage schedule");
#pragma unroll
  for (int s = 0; s < PSTAGES - 1; ++s) t.stage(L.s[s], min(s, nk - 1));
  int kt = 0;
  for (; kt + 4 <= nk; kt += 4) {
    t.template step<0, 3>(L, kt);
    t.template step<1, 0>(L, kt + 1);
    t.template step<2, 1>(L, kt + 2);
    t.template step<3, 2>(L, kt + 3);
  }
  const int rem = nk - kt;
  if (rem > 0) t.template step<0, 3>(L, kt);
  if (rem > 1) t.template step<1, 0>(L, kt + 1);
  if (rem > 2) t.template step<2, 1>(L, kt + 2);
  PWAIT_VM(0);   // no staging in flight when the workgroup moves on
  if (!t.live) return;
  const int M = SYRK ? p.ms : p.mr, N = SYRK ? p.ns : p.nr;
  double* Cm = (SYRK ? p.Atr : p.Brow) + boff;
  // 16x16 f64 block layout: column lane % 16, row lane / 16 + 4 e.  Per 16-row block the 16
  // loads are issued together (clamped in-bounds addresses), then the 16 stores.
  const int ib = i0 + 32 * t.wr + t.g, jb = j0 + 64 * t.wc + t.r;
  const bool full = (i0 + PT <= M) && (j0 + PT <= N);
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    double cv[4][4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = min(ib + 16 * rb + 4 * e, M - 1), j = min(jb + 16 * cb, N - 1);
        cv[cb][e] = Cm[(int64_t)i * p.ld + j];
      }
    if (full) {   // interior tile: no per-element branches, so the stores wait once
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          Cm[(int64_t)(ib + 16 * rb + 4 * e) * p.ld + jb + 16 * cb] = cv[cb][e] - t.acc[rb][cb][e];
    } else {
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = ib + 16 * rb + 4 * e, j = jb + 16 * cb;
          if (i < M && j < N) Cm[(int64_t)i * p.ld + j] = cv[cb][e] - t.acc[rb][cb][e];
        }
    }
  }
}

// Tile order.  Tiles are walked in bands of `band` tile rows, column by column inside a band
// (then the band's rows): a column operand tile (128 panel rows x K) then serves `band` output
// tiles while it is in L2, and the band's row operand (band x 128 x K doubles: 2 MB, 8 rows at
// K = 256 or 4 at K = 512) stays there for the whole band.  Row-major order re-fetched every
// column operand once per tile row: 3x the algorithmic bytes at C = 28672.
__host__ __device__ constexpr int panel_band(int K) { return K > 256 ? 4 : 8; }

// u-th tile of the lower trapezoid {(ti, tj): tj <= ti < ntr, tj < ntc} in band order.
__device__ __forceinline__ void lower_tile_banded(int u, int ntr, int ntc, int PBAND, int& ti, int& tj) {
  int b0 = 0;
  for (;;) {
    const int h = min(PBAND, ntr - b0);
    const int ce = min(b0 + h, ntc);
    int cnt = min(b0, ntc) * h;                 // columns left of the band: h rows each
    for (int c = b0; c < ce; ++c) cnt += b0 + h - c;
    if (u < cnt || b0 + h >= ntr) break;
    u -= cnt;
    b0 += h;
  }
  const int h = min(PBAND, ntr - b0);
  const int full = min(b0, ntc) * h;
  if (u < full) {
    tj = u / h;
    ti = b0 + u % h;
    return;
  }
  u -= full;
  for (int c = b0;; ++c) {           // column c holds rows c .. b0 + h - 1 of the band
    const int k = b0 + h - c;
    if (u < k) {
      tj = c;
      ti = c + u;
      return;
    }
    u -= k;
  }
}

// u-th tile of an nr x nc grid in band order.
__device__ __forceinline__ void rect_tile_banded(int u, int nr, int nc, int PBAND, int& ti, int& tj) {
  const int band = u / (PBAND * nc);
  const int b0 = band * PBAND;
  const int h = min(PBAND, nr - b0);
  const int v = u - b0 * nc;
  tj = v / h;
  ti = b0 + v % h;
}

constexpr int PTHREADS = 512;
__global__ __launch_bounds__(PTHREADS, 2) void k_panel_update(PanelArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t lds0[PSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds1[PSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds2[PSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds3[PSTAGE];
  const PStages L{{lds0, lds1, lds2, lds3}};
  // XCD-aware order: workgroup b runs on XCD b % 8; each XCD takes a contiguous range of
  // tiles, so tiles that share panel rows meet in one L2.
  const int b = blockIdx.x;
  const int per = p.total / 8, rem8 = p.total % 8;
  const int xcd = b % 8, idx = b / 8;
  const int t = (xcd < rem8) ? xcd * (per + 1) + idx : rem8 * (per + 1) + (xcd - rem8) * per + idx;
  if (t >= p.total) return;
  const int bz = t / p.per_batch, u = t % p.per_batch;
  if (p.info[bz]) return;
  const int64_t boff = (int64_t)bz * p.ws;
  int ti, tj;
  if (u < p.nsy) {
    lower_tile_banded(u, p.ntr, p.ntc, panel_band(p.K), ti, tj);
    panel_tile<true>(p, boff, ti, tj, L);
  } else {
    rect_tile_banded(u - p.nsy, p.nrr, p.nrc, panel_band(p.K), ti, tj);
    panel_tile<false>(p, boff, ti, tj, L);
  }
}

}  // namespace

// One k_panel_update launch over nb batch entries (see PanelArgs).  Requires C even and K a
// multiple of PKS; returns false (nothing launched) otherwise.
inline bool launch_panel(const double* Lp, const double* X, double* Atr, double* Brow, int C, int K,
                         int ms, int ns, int mr, int nr, int64_t ws, const int* info, int nb,
                         hipStream_t s) {
  if ((C & 1) || K % PKS || K <= 0) return false;
  PanelArgs pa;
  pa.Lp = Lp;
  pa.X = X;
  pa.Atr = Atr;
  pa.Brow = Brow;
  pa.ld = C;
  pa.K = K;
  pa.ms = ms;
  pa.ns = ns;
  pa.mr = mr;
  pa.nr = nr;
  pa.ntr = ms > 0 ? (ms + PT - 1) / PT : 0;
  pa.ntc = ns > 0 ? (ns + PT - 1) / PT : 0;
  pa.nsy = 0;
  for (int ti = 0; ti < pa.ntr; ++ti) pa.nsy += (ti + 1 < pa.ntc) ? ti + 1 : pa.ntc;
  pa.nrr = (mr > 0 && nr > 0) ? (mr + PT - 1) / PT : 0;
  pa.nrc = (mr > 0 && nr > 0) ? (nr + PT - 1) / PT : 0;
  pa.per_batch = pa.nsy + pa.nrr * pa.nrc;
  pa.ws = ws;
  pa.info = info;
  pa.total = pa.per_batch * nb;
  if (pa.total > 0) hipLaunchKernelGGL(k_panel_update, dim3(pa.total), dim3(PTHREADS), 0, s, pa);
  return true;
}

extern "C" int64_t rq_chol_workspace_bytes(int C) {
  if (C <= 0) return -1;
  return ((int64_t)2 * C * C + (int64_t)NB * NB) * (int64_t)sizeof(double);
}

extern "C" int rq_chol_hinv_attempt(float* H_work, int C, int nb, const double* damp_percent,
                                    void* workspace, float* Hinv, float* Hinv_init,
                                    float* Hinv_diag, int* info,
                                    void* stream) {
  using namespace rq;
  if (!H_work || !workspace || !Hinv || !info || !damp_percent || C <= 0 || nb <= 0 ||
      nb > MAXBATCH)
    return RQ_EINVAL;
  BatchCfg cfg;
  int n_active = 0;
  for (int b = 0; b < MAXBATCH; ++b) {
    cfg.damp[b] = 0.0f;
    cfg.active[b] = 0;
  }
  for (int b = 0; b < nb; ++b) {
    const double p = damp_percent[b];
    if (p > 0) {
      if (!(p < 1.0)) return RQ_EINVAL;
      cfg.damp[b] = (float)p;   // torch multiplies the fp32 mean by the scalar in fp32
      cfg.active[b] = 1;
      ++n_active;
    }
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_init_info, dim3(1), dim3(MAXBATCH), 0, s, info, nb, cfg);
  RQ_CHECK_LAUNCH();
  if (n_active == 0) return RQ_OK;
  const int64_t ws = 2 * (int64_t)C * C + (int64_t)NB * NB;   // doubles per batch entry
  double* A = reinterpret_cast<double*>(workspace);
  double* Linv = A + (int64_t)C * C;
  const dim3 blk(256);
  const dim3 gcol((C + 255) / 256, C < 1024 ? C : 1024, nb);

  hipLaunchKernelGGL(k_damp, dim3(nb), blk, 0, s, H_work, C, cfg, info);
  hipLaunchKernelGGL(k_reverse_to_f64, gcol, blk, 0, s, H_work, C, A, Linv, ws, info);
  RQ_CHECK_LAUNCH();

  auto batched = [&](GemmArgs<double> g) {
    g.abort_flag = info;
    g.sA = ws;
    g.sB = ws;
    g.sC = ws;
    return g;
  };
  // Two-level blocking: outer panels of NBW columns, factored in NB-wide steps whose updates
  // stay inside the panel; the trailing matrix (and the rows of L^-1 below the panel) get
  // one rank-NBW update per panel, so the big updates read and write the trailing matrix
  // NBW / NB times less often.
  const int NBW = panel_width(C);
  int rc;
  // The factorisation of columns [k, pe): per NB block the diagonal factor and inverse, the
  // block column of L and row block of L^-1, and the update of the later columns up to pe.
  auto factor_cols = [&](int k, int pe) -> int {
    for (int j = k; j < pe; j += NB) {
      const int jb = (pe - j < NB) ? (pe - j) : NB;
      const int below = C - j - jb;                      // rows below this block (whole matrix)
      const int pend = pe - j - jb;                      // panel columns right of this block
      // one launch: T = L_jj^-1, then L_ij = A_ij T^T (in place, every row below the block) and
      // X_j[:, 0:j] = T B_j[:, 0:j] (in place, row block j of L^-1)
      StepArgs sa{A, Linv, C, j, jb, (below + NB - 1) / NB, (j + NB - 1) / NB, ws, info};
      const int ntiles = sa.n1 + sa.n2;
      const int per_entry = std::max(1, std::min(ntiles, std::max(1, STEP_SLOTS / nb)));
      hipLaunchKernelGGL(k_chol_step, dim3(per_entry, 1, nb), dim3(CD_THREADS), 0, s, sa);
      RQ_CHECK_LAUNCH();
      int r;
      // one launch, inside [k, pe): A[j+jb:, j+jb:pe] -= L[j+jb:, j] L[j+jb:pe, j]^T (lower
      // tiles) and those rows of L^-1: B[j+jb:pe, 0:j+jb] -= L[j+jb:pe, j] X_j.  On the 128-tile
      // panel kernel when [k, pe) is wider than 256 (up to 448 columns); the narrower updates
      // have too few 128-tiles and run faster on the 64-tile GEMM.
      if (pend > 0 && pe - k > 256 && launch_panel(A + (int64_t)(j + jb) * C + j, Linv + (int64_t)j * C,
                                   A + (int64_t)(j + jb) * C + (j + jb), Linv + (int64_t)(j + jb) * C,
                                   C, jb, below, pend, pend, j + jb, ws, info, nb, s)) {
        RQ_CHECK_LAUNCH();
      } else if (pend > 0) {
        GemmArgs<double> h = batched(gemm_args<double>(A + (int64_t)(j + jb) * C + j, C,
                                                       A + (int64_t)(j + jb) * C + j, C,
                                                       A + (int64_t)(j + jb) * C + (j + jb), C, below,
                                                       pend, jb, -1.0, EPI_ACCUM));
        h.lower_only = 1;
        GemmArgs<double> g = batched(gemm_args<double>(A + (int64_t)(j + jb) * C + j, C,
                                                       Linv + (int64_t)j * C, C,
                                                       Linv + (int64_t)(j + jb) * C, C, pend, j + jb,
                                                       jb, -1.0, EPI_ACCUM));
        if ((r = launch_gemm_pair(h, g, s, nb))) return r;
      }
    }
    return RQ_OK;
  };
  // The update by panel [k, k + kw) of the trailing rows r0 ..: A[r0:r0+ms, r0:r0+ns] -=
  // L[r0:, k:k+kw] L[r0:, k:k+kw]^T (lower tiles) and B[r0:r0+mr, 0:nr] -= L[r0:r0+mr, k:k+kw]
  // X[k:k+kw, 0:nr], on the 128-tile panel kernel, or on the 64-tile GEMM when the panel kernel
  // does not take the shape.
  auto trailing = [&](int k, int kw, int r0, int ms, int ns, int mr, int nr, hipStream_t st) -> int {
    if (launch_panel(A + (int64_t)r0 * C + k, Linv + (int64_t)k * C, A + (int64_t)r0 * C + r0,
                               Linv + (int64_t)r0 * C, C, kw, ms, ns, mr, nr, ws, info, nb, st)) {
      RQ_CHECK_LAUNCH();
      return RQ_OK;
    }
    GemmArgs<double> h = batched(gemm_args<double>(A + (int64_t)r0 * C + k, C, A + (int64_t)r0 * C + k, C,
                                                   A + (int64_t)r0 * C + r0, C, ms, ns, kw, -1.0, EPI_ACCUM));
    h.lower_only = 1;
    GemmArgs<double> g = batched(gemm_args<double>(A + (int64_t)r0 * C + k, C, Linv + (int64_t)k * C, C,
                                                   Linv + (int64_t)r0 * C, C, mr, nr, kw, -1.0, EPI_ACCUM));
    return launch_gemm_pair(h, g, st, nb);
  };

  // One panel [k, pe).  A 512-wide panel is factored as two 256-wide halves: the first half's
  // blocks update only its own later columns (rank 64 each), one rank-256 update then carries
  // the first half into the second half's columns (all rows below) and rows of L^-1, and the
  // second half follows.  The same operations as one pass over the panel, grouped so that
  // more of the in-panel work runs at the rank-256 rate (C = 14336, 4 subgroups: 143.3 ->
  // 141.0 ms per chain).
  auto factor_panel = [&](int k, int pe) -> int {
    if (pe - k > 256) {
      const int h = k + 256;
      int r;
      if ((r = factor_cols(k, h))) return r;
      if ((r = trailing(k, 256, h, C - h, pe - h, pe - h, h, s))) return r;
      return factor_cols(h, pe);
    }
    return factor_cols(k, pe);
  };
  // Look-ahead over two streams, for the 512-wide panels (C >= 8192: at C = 4096 the overlap
  // gains less than the latency-bound factorisation kernels lose while the far update holds the
  // CUs).  After panel p the trailing update is split: the near part
  // (the next panel's columns, all rows below, and its rows of L^-1) runs on the caller's
  // stream, and the next panel's factorisation follows it at once; the far part (the columns
  // and L^-1 rows past the next panel) runs on the side stream meanwhile.  The near part of
  // panel p+1 waits for the far part of panel p, which updated the same columns; a far part
  // starts after the panel that produced its operands and after the previous far part.  The
  // two parts write disjoint tiles and read only finished panels.
  std::unique_lock<std::mutex> side_lock;
  RqSideJoin join;
  join.s = s;
  for (int k = 0; k < C; k += NBW) {
    const int kw = (C - k < NBW) ? (C - k) : NBW;
    const int pe = k + kw;                               // panel end
    if ((rc = factor_panel(k, pe))) return rc;
    const int rest = C - pe;
    if (rest <= 0) break;
    const int w2 = (rest < NBW) ? rest : NBW;            // the next panel's width
    const int rest2 = rest - w2;
    if (rest2 > 0 && NBW > 256) {
      if (!join.sd && (rc = rq_side_stream(&join.sd, side_lock))) return rc;
      RqSide* sd = join.sd;
      if (hipEventRecord(sd->fork, s) != hipSuccess) return RQ_EHIP;
      if (join.busy && hipStreamWaitEvent(s, sd->join, 0) != hipSuccess) return RQ_EHIP;
      if (hipStreamWaitEvent(sd->s, sd->fork, 0) != hipSuccess) return RQ_EHIP;
      if ((rc = trailing(k, kw, pe + w2, rest2, rest2, rest2, pe, sd->s))) return rc;
      if (hipEventRecord(sd->join, sd->s) != hipSuccess) return RQ_EHIP;
      join.busy = true;
      if ((rc = trailing(k, kw, pe, rest, w2, w2, pe, s))) return rc;
    } else {
      if (join.busy) {
        if (hipStreamWaitEvent(s, join.sd->join, 0) != hipSuccess) return RQ_EHIP;
        join.busy = false;
      }
      if ((rc = trailing(k, kw, pe, rest, rest, rest, pe, s))) return rc;
    }
  }
  if (join.busy) {
    if (hipStreamWaitEvent(s, join.sd->join, 0) != hipSuccess) return RQ_EHIP;
    join.busy = false;
  }
  hipLaunchKernelGGL(k_output_upper, gcol, blk, 0, s, Linv, C, Hinv, ws, info);
  RQ_CHECK_LAUNCH();
  if (Hinv_diag) {
    // partial column norms in A (free once the factorisation is done)
    const int nch = diag_chunks(C);
    const dim3 gd((C + 255) / 256, nch, nb), gf((C + 255) / 256, 1, nb);
    hipLaunchKernelGGL(k_diag_partial, gd, blk, 0, s, Linv, C, A, ws, info);
    hipLaunchKernelGGL(k_diag_final, gf, blk, 0, s, A, C, nch, ws, Hinv_diag, info);
    RQ_CHECK_LAUNCH();
  }
  if (Hinv_init) {
    // M = Linv^T Linv (lower tiles) into A, then Hinv_init = P M P.
    GemmArgs<double> g = batched(gemm_args<double>(Linv, C, Linv, C, A, C, C, C, C, 1.0, EPI_STORE));
    g.krange = KR_AB_LOWER;
    g.lower_only = 1;
    rc = launch_gemm(g, true, false, s, nb);
    if (rc) return rc;
    hipLaunchKernelGGL(k_output_full, gcol, blk, 0, s, A, C, Hinv_init, ws, info);
    RQ_CHECK_LAUNCH();
  }
  return RQ_OK;
}
