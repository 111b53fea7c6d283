// Damped Cholesky chain (GPTQPlus._compute_hessian_inverse_with_fallback,
// gptq_utils/gptq_plus_utils.py:494-561).
//
// The reference computes chol(H) -> cholesky_inverse -> chol(H^-1, upper) in fp32.  Here the
// upper factor U of H^-1 (U^T U = H^-1) is obtained with ONE factorisation: with P the
// index-reversal permutation and L L^T = P H P,  U = P L^-1 P.  The factorisation and the
// inverse L^-1 run together in one right-looking blocked pass in fp64 (64-wide blocks
// inside 256-wide panels, 512-wide from C = 8192):
//   per block k:  L_kk = chol(A_kk) and T = L_kk^-1 (k_chol_diag, one workgroup per matrix),
//                 L_ik = A_ik T^T,  X_k = T B_k  (row block k of L^-1),
//                 A_ij -= L_ik L_jk^T (lower tiles),  B_i -= L_ik X_k   (fp64 MFMA GEMMs),
// where B accumulates I - sum_m L_im X_m.  The updates of the trailing matrix and of the rows
// of B below a panel are applied once per panel (rank 256 / 512) instead of once per block,
// by k_panel_update (128x128 tiles, direct global->LDS staging).  H^-1 itself (Hinv_init) is
// P (L^-T L^-1) P and is only formed when asked for; its diagonal (all that the GPTQ+ step
// size needs of it) comes from the column norms of L^-1.  A non-positive or non-finite pivot, or
// a non-finite result, raises the device `info` flag; later kernels of the same attempt exit
// early.
#include "gemm_tile.h"

namespace {

constexpr int NB = 64;     // diagonal block (factored and inverted by one workgroup)
constexpr int CG = 4;      // columns factored per barrier in the diagonal block
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

// 1/sqrt(d) and sqrt(d) in fp64 from the hardware estimate and two Newton steps
// y <- y (3 - d y^2) / 2 (the error squares each step: well below fp64 rounding after two).
__device__ __forceinline__ void rsqrt_newton(double d, double& rs, double& sq) {
  double y = __builtin_amdgcn_rsq(d);
  const double h = 0.5 * d;
  y = y * __builtin_fma(-h * y, y, 1.5);
  y = y * __builtin_fma(-h * y, y, 1.5);
  rs = y;
  sq = d * y;
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Sum of a double over the 4 lanes of a quad (DPP quad_perm moves, no LDS).
template <int CTRL>
__device__ __forceinline__ double quad_mov_f64(double v) {
  const uint64_t u = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double quad_sum_f64(double v) {
  v = v + quad_mov_f64<0xB1>(v);   // lanes [1, 0, 3, 2]
  return v + quad_mov_f64<0x4E>(v);   // lanes [2, 3, 0, 1]
}

// Factor the nb x nb diagonal block of A at (k, k) and invert it; one workgroup of 4 waves per
// batch entry (rows >= nb are identity padding).
//  - Factor: lane r of wave w holds L[r][16w .. 16w+15] (16 registers).  Columns go in groups
//    of CG = 4, all held by one wave.  For each column j of the group that wave takes the pivot
//    from lane j (readlane), forms 1/sqrt and sqrt, scales its column (L[r][j], zero for
//    r <= j) and subtracts L[r][j] L[l][j] from the group's later columns l itself (L[l][j] by
//    readlane); then it publishes the group's columns in `col` (two buffers, alternating by
//    group, so one barrier per group orders each write after the previous reads), and every
//    wave subtracts L[r][j] L[l][j], j in the group in order, from its other columns l (col is
//    zero at l <= j, so finished columns stay as they are).  Every entry sees the same fused
//    multiply-adds in the same order as with one column per barrier.
//  - Inverse: lane quad c of the workgroup computes column c of T = L^-1 by forward
//    substitution t[i] = (delta_ic - sum_{m<i} L[i][m] t[m]) / L[i][i]; lane q of the quad
//    holds the rows m = 4p + q and its part of each dot product, and the quad adds the four
//    parts with DPP moves.  L is staged in LDS column-interleaved (element (i, 4p + q) at
//    i * LS + 16 q + p), so a lane reads its operands of a row in 16-byte pieces, and the
//    lanes of one q in a wave all read the same address (broadcast).
// Writes T (lower, exact zeros above) to Tbuf and to Linv's diagonal block.
constexpr int CD_THREADS = 256;
__global__ __launch_bounds__(CD_THREADS) void k_chol_diag(const double* __restrict__ A, int C, int k,
                                                          int nb, double* __restrict__ Tbuf,
                                                          double* __restrict__ Linv, int64_t ws,
                                                          int* info_all) {
  constexpr int LS = NB + 2;                        // LDS row stride (16-byte aligned rows)
  __shared__ __attribute__((aligned(16))) double S[NB * LS];
  __shared__ __attribute__((aligned(16))) double col[2][CG][NB];
  __shared__ double dinv[NB];   // 1 / L[j][j]; NaN marks a failed pivot
  const int b = blockIdx.x;
  int* info = info_all + b;
  if (*info) return;
  A += b * ws;
  Tbuf += b * ws;
  Linv += b * ws;
  const int tid = threadIdx.x;
  const int r = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // columns 16 wave .. 16 wave + 15 of row r of the block's lower triangle (zeros above,
  // identity on the padding rows).  Only rows < nb and columns < nb are read: a ragged last
  // block reads with a clamped column index, and the mask clears those columns (they lie
  // above the diagonal of every row that is read).  A full block with C even (k is a
  // multiple of NB) has 16-byte aligned rows.
  const int c0 = 16 * wave;
  double a[16];
  if (r < nb) {
    const double* rowp = A + (int64_t)(k + r) * C + k + c0;
    if (nb == NB && (C & 1) == 0) {
      const double2* row = reinterpret_cast<const double2*>(rowp);
#pragma unroll
      for (int q = 0; q < 16; q += 2) {
        const double2 v = row[q / 2];
        a[q] = v.x;
        a[q + 1] = v.y;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) a[q] = A[(int64_t)(k + r) * C + k + min(c0 + q, nb - 1)];
    }
#pragma unroll
    for (int q = 0; q < 16; ++q)
      if (c0 + q > r) a[q] = 0.0;
  } else {
#pragma unroll
    for (int q = 0; q < 16; ++q) a[q] = (c0 + q == r) ? 1.0 : 0.0;
  }
  __syncthreads();

  bool fail = false;
#pragma unroll
  for (int g = 0; g < NB / CG; ++g) {
    const int j0 = CG * g, jw = j0 / 16, jq0 = j0 % 16;
    double (*cg)[NB] = col[g & 1];
    if (wave == jw) {
#pragma unroll
      for (int u = 0; u < CG; ++u) {
        const int j = j0 + u, jq = jq0 + u;
        const double d = readlane_f64(a[jq], j);     // uniform pivot
        double rd = 0.0, sq = 0.0;
        const bool ok = d > 0.0 && rq_isfinite(d);
        if (ok) rsqrt_newton(d, rd, sq);
        const double lrj = (r > j) ? a[jq] * rd : 0.0;  // L[r][j]
        a[jq] = (r == j) ? sq : lrj;
        cg[u][r] = lrj;
        if (r == 0) dinv[j] = ok ? rd : __builtin_nan("");
#pragma unroll
        for (int v = u + 1; v < CG; ++v)                  // the group's later columns
          a[jq0 + v] = __builtin_fma(-lrj, readlane_f64(lrj, j0 + v), a[jq0 + v]);
      }
    }
    __syncthreads();
    // dinv[j] is written once, before this barrier: every wave reads the same verdict.  The
    // columns are read before the verdict is tested (the reads are in bounds either way).
    bool bad = false;
    double m[CG], cv[CG][16];
#pragma unroll
    for (int u = 0; u < CG; ++u) {
      const double dj = dinv[j0 + u];
      bad |= !(dj == dj);
      m[u] = cg[u][r];
#pragma unroll
      for (int q = 0; q < 16; ++q) cv[u][q] = cg[u][c0 + q];
    }
    if (bad) {
      fail = true;
      break;
    }
    // q-major, so the next group's columns are done first; the group's own columns were
    // updated by their wave above
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      const bool own = (q >= jq0 && q < jq0 + CG) && wave == jw;
#pragma unroll
      for (int u = 0; u < CG; ++u) {
        const double nv = __builtin_fma(-m[u], cv[u][q], a[q]);
        a[q] = own ? a[q] : nv;
      }
    }
  }
  if (fail) {
    if (tid == 0) atomicExch(info, 1);
    return;
  }
  // L into LDS, column-interleaved; entries above the diagonal are zero
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int c = c0 + q;
    S[r * LS + 16 * (c & 3) + (c >> 2)] = (c <= r) ? a[q] : 0.0;
  }
  __syncthreads();

  const int cc = tid >> 2, qq = tid & 3;
  const double* Sq = S + 16 * qq;
  double t[16];
#pragma unroll
  for (int p = 0; p < 16; ++p) t[p] = 0.0;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    // rows m = 4p + qq < i; L[i][m] = 0 for m >= i, so p runs to (i - 1) / 4 for every lane
    double part = 0.0;
    if (i > 0) {
      const int np = (i - 1) / 4 + 1;
      double s2[2] = {0.0, 0.0};
#pragma unroll
      for (int p = 0; p < np; p += 2) {
        const double2 l = *reinterpret_cast<const double2*>(Sq + i * LS + p);
        s2[0] = __builtin_fma(l.x, t[p], s2[0]);
        if (p + 1 < np) s2[1] = __builtin_fma(l.y, t[p + 1], s2[1]);
      }
      part = s2[0] + s2[1];
    }
    const double di = dinv[i];
    const double tot = quad_sum_f64(part);
    const double ti = (((i == cc) ? 1.0 : 0.0) - tot) * di;
    t[i >> 2] = ((i & 3) == qq) ? ti : t[i >> 2];   // a select, not a branch
  }
  // t[p] = T[4p + qq][cc]
#pragma unroll
  for (int p = 0; p < 16; ++p) Tbuf[(4 * p + qq) * NB + cc] = t[p];
  if (cc < nb) {
#pragma unroll
    for (int p = 0; p < 16; ++p)
      if (4 * p + qq < nb) Linv[(int64_t)(k + 4 * p + qq) * C + (k + cc)] = t[p];
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
    __builtin_amdgcn_s_barrier();
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
  double* Tbuf = Linv + (int64_t)C * C;
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
  for (int k = 0; k < C; k += NBW) {
    const int kw = (C - k < NBW) ? (C - k) : NBW;
    const int pe = k + kw;                               // panel end
    for (int j = k; j < pe; j += NB) {
      const int jb = (pe - j < NB) ? (pe - j) : NB;
      const int below = C - j - jb;                      // rows below this block (whole matrix)
      const int pend = pe - j - jb;                      // panel columns right of this block
      hipLaunchKernelGGL(k_chol_diag, dim3(nb), dim3(CD_THREADS), 0, s, A, C, j, jb, Tbuf, Linv, ws, info);
      RQ_CHECK_LAUNCH();
      int rc;
      // one launch: L_ij = A_ij T^T (in place, every row below the block) and
      // X_j[:, 0:j] = T B_j[:, 0:j] (in place, row block j of L^-1)
      GemmArgs<double> lij = batched(gemm_args<double>(A + (int64_t)(j + jb) * C + j, C, Tbuf, NB,
                                                       A + (int64_t)(j + jb) * C + j, C, below, jb, jb,
                                                       1.0, EPI_STORE));
      GemmArgs<double> xj = batched(gemm_args<double>(Tbuf, NB, Linv + (int64_t)j * C, C,
                                                      Linv + (int64_t)j * C, C, jb, j, jb, 1.0, EPI_STORE));
      if ((rc = launch_gemm_pair(lij, xj, s, nb))) return rc;
      // one launch, inside the panel: A[j+jb:, j+jb:pe] -= L[j+jb:, j] L[j+jb:pe, j]^T (lower
      // tiles) and the panel rows of L^-1: B[j+jb:pe, 0:j+jb] -= L[j+jb:pe, j] X_j.  On the
      // 128-tile panel kernel with 512-wide panels (up to 448 columns); the narrower updates of
      // 256-wide panels have too few 128-tiles and run faster on the 64-tile GEMM.
      if (pend > 0 && NBW > 256 && launch_panel(A + (int64_t)(j + jb) * C + j, Linv + (int64_t)j * C,
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
        if ((rc = launch_gemm_pair(h, g, s, nb))) return rc;
      }
    }
    const int rest = C - pe;
    // one launch: the trailing matrix A[pe:, pe:] -= L[pe:, k:pe] L[pe:, k:pe]^T (lower tiles,
    // K = kw) and the rows of L^-1 below the panel: B[pe:, 0:pe] -= L[pe:, k:pe] X[k:pe, 0:pe]
    if (rest > 0 && launch_panel(A + (int64_t)pe * C + k, Linv + (int64_t)k * C, A + (int64_t)pe * C + pe,
                                 Linv + (int64_t)pe * C, C, kw, rest, rest, rest, pe, ws, info, nb, s)) {
      RQ_CHECK_LAUNCH();
    } else if (rest > 0) {
      // the same two updates on the 64-tile GEMM (odd C, or a panel width not a multiple of 8)
      GemmArgs<double> h = batched(gemm_args<double>(A + (int64_t)pe * C + k, C, A + (int64_t)pe * C + k,
                                                     C, A + (int64_t)pe * C + pe, C, rest, rest, kw,
                                                     -1.0, EPI_ACCUM));
      h.lower_only = 1;
      GemmArgs<double> g = batched(gemm_args<double>(A + (int64_t)pe * C + k, C, Linv + (int64_t)k * C,
                                                     C, Linv + (int64_t)pe * C, C, rest, pe, kw, -1.0,
                                                     EPI_ACCUM));
      int rc;
      if ((rc = launch_gemm_pair(h, g, s, nb))) return rc;
    }
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
    int rc = launch_gemm(g, true, false, s, nb);
    if (rc) return rc;
    hipLaunchKernelGGL(k_output_full, gcol, blk, 0, s, A, C, Hinv_init, ws, info);
    RQ_CHECK_LAUNCH();
  }
  return RQ_OK;
}
