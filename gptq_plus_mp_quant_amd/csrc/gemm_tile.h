// 64x64-tile MFMA GEMM shared by the Cholesky chain (fp64) and the GPTQ+ setup GEMMs (fp32).
//
//   C[i, j] (op)= alpha * sum_k A(i, k) B(k, j)        i < M, j < N, k in [k_lo(tile), k_hi(tile))
//   A(i, k) = TA ? A[k*lda + i] : A[i*lda + k]        B(k, j) = TB ? B[j*ldb + k] : B[k*ldb + j]
//
// 256 threads = 4 waves in a 2x2 arrangement, 32x32 per wave as 2x2 blocks of the 16x16x4
// MFMA (v_mfma_f32_16x16x4f32 / v_mfma_f64_16x16x4f64).  K advances in slabs of 32 through
// LDS; the next slab is fetched into registers (16-byte loads inside the matrix) while the
// current one is multiplied.
// Triangular operands are handled by restricting the K range per output tile (the invalid
// triangle of every operand used here is stored as explicit zeros).
#pragma once
#include "rq_common.h"

namespace rq {

template <typename T>
struct Mfma16;
// Output element e of a lane: column lane % 16, row row(lane, e).  The fp32 op returns four
// consecutive rows per lane group, the fp64 op interleaves them (checked on gfx950).
template <>
struct Mfma16<float> {
  using acc_t = floatx4;
  static __device__ __forceinline__ int row(int lane, int e) { return 4 * (lane >> 4) + e; }
  static __device__ __forceinline__ acc_t op(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma16<double> {
  using acc_t = doublex4;
  static __device__ __forceinline__ int row(int lane, int e) { return (lane >> 4) + 4 * e; }
  static __device__ __forceinline__ acc_t op(double a, double b, acc_t c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
};

// K-range restriction per output tile (tile origin i0, j0; 64 wide).
enum KRange : int {
  KR_FULL = 0,
  KR_B_UPPER = 1,   // B(k, j) == 0 for k > j   -> k < j0 + 64
  KR_B_LOWER = 2,   // B(k, j) == 0 for k < j   -> k >= j0
  KR_AB_LOWER = 3,  // A(i,k)==0 for k<i and B(k,j)==0 for k<j -> k >= max(i0, j0)
};

// Epilogue modes.
enum Epi : int {
  EPI_STORE = 0,     // C = alpha * acc
  EPI_ACCUM = 1,     // C = C + alpha * acc
};

template <typename T>
struct GemmArgs {
  const T* A;
  int64_t lda;
  const T* B;
  int64_t ldb;
  T* Cm;
  int64_t ldc;
  int M, N, K;
  T alpha;
  int epi;
  int krange;
  int lower_only;            // skip output tiles strictly above the diagonal
  const T* row_scale;        // optional epilogue factor: row_scale[row_bcast ? 0 : i]
  int row_bcast;
  int* nz_flag;              // optional: set to 1 when any stored value is non-zero or NaN
  const int* skip_if_zero;   // optional: when *skip_if_zero == 0 store zeros and return
  const int* abort_flag;     // optional: when abort_flag[batch] != 0 return immediately
  int64_t sA, sB, sC;        // element strides between batch entries (grid z = batch)
  int vec;                   // set by launch_gemm: A / B rows and batch strides 16-byte aligned
};

constexpr int GT = 64;
constexpr int GKT = 32;
constexpr int GCH = 8;   // consecutive elements per thread in a slab fetch
// LDS row padding of the 64-wide slabs.  fp64: a row of 65 doubles (130 dwords, 2 banks past
// a multiple of 32) spreads every access pattern below evenly over the 32 banks: the MFMA
// operand reads (4 rows x 16 consecutive doubles per instruction) and all four slab stores
// (8 rows x 8 threads 8 doubles apart, or 4 rows x 16 consecutive threads).  fp32 keeps 68.
template <typename T>
struct GPad {
  static constexpr int v = 4;
};
template <>
struct GPad<double> {
  static constexpr int v = 1;
};

template <typename T>
__device__ __forceinline__ void load_chunk(const T* __restrict__ src, bool vec, T (&r)[GCH]) {
  if (vec) {   // 16-byte aligned, fully in bounds
    const uint4* q = reinterpret_cast<const uint4*>(src);
    constexpr int NV = GCH * sizeof(T) / 16;
    uint4 v[NV];
#pragma unroll
    for (int e = 0; e < NV; ++e) v[e] = q[e];
#pragma unroll
    for (int e = 0; e < GCH; ++e) r[e] = reinterpret_cast<const T*>(v)[e];
  }
}

// One 64x64 output tile (row tile ti, column tile tj) of batch entry bz.
template <typename T, bool TA, bool TB>
__device__ __forceinline__ void gemm_tile_body(GemmArgs<T> p, int ti, int tj, int bz,
                                               T (*__restrict__ As)[GT + GPad<T>::v],
                                               T (*__restrict__ Bs)[GT + GPad<T>::v]) {
  using acc_t = typename Mfma16<T>::acc_t;
  if (p.abort_flag && p.abort_flag[bz]) return;
  p.A += bz * p.sA;
  p.B += bz * p.sB;
  p.Cm += bz * p.sC;
  if (p.lower_only && tj > ti) return;
  const int i0 = ti * GT, j0 = tj * GT;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;

  if (p.skip_if_zero && *p.skip_if_zero == 0) {
    for (int e = tid; e < GT * GT; e += 256) {
      const int i = i0 + e / GT, j = j0 + e % GT;
      if (i < p.M && j < p.N) p.Cm[(int64_t)i * p.ldc + j] = T(0);
    }
    return;
  }

  int k_lo = 0, k_hi = p.K;
  if (p.krange == KR_B_UPPER) k_hi = min(p.K, j0 + GT);
  else if (p.krange == KR_B_LOWER) k_lo = j0;
  else if (p.krange == KR_AB_LOWER) k_lo = max(i0, j0);
  k_lo = (k_lo / GKT) * GKT;

  acc_t acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[a][b][e] = T(0);

  // Slab fetch: A 64 (i) x 32 (k), B 32 (k) x 64 (j), 8 consecutive elements per thread,
  // as 16-byte loads when the slab is inside the matrix and rows are 16-byte aligned.
  const bool rows_in = (i0 + GT <= p.M) && (j0 + GT <= p.N);
  T ra[GCH], rb[GCH];
  auto fetch = [&](int k0) {
    const bool vec = p.vec && rows_in && (k0 + GKT <= k_hi);
    if (!TA) {  // A[i][k]: row i = tid / 4, k chunk (tid % 4) * 8
      const int i = i0 + (tid >> 2), kq = k0 + (tid & 3) * GCH;
      const T* src = p.A + (int64_t)i * p.lda + kq;
      load_chunk<T>(src, vec, ra);
      if (!vec)
#pragma unroll
        for (int e = 0; e < GCH; ++e) ra[e] = (i < p.M && kq + e < k_hi) ? src[e] : T(0);
    } else {    // A[k][i]: k = tid / 8, i chunk (tid % 8) * 8
      const int k = k0 + (tid >> 3), iq = i0 + (tid & 7) * GCH;
      const T* src = p.A + (int64_t)k * p.lda + iq;
      load_chunk<T>(src, vec, ra);
      if (!vec)
#pragma unroll
        for (int e = 0; e < GCH; ++e) ra[e] = (k < k_hi && iq + e < p.M) ? src[e] : T(0);
    }
    if (!TB) {  // B[k][j]: k = tid / 8, j chunk (tid % 8) * 8
      const int k = k0 + (tid >> 3), jq = j0 + (tid & 7) * GCH;
      const T* src = p.B + (int64_t)k * p.ldb + jq;
      load_chunk<T>(src, vec, rb);
      if (!vec)
#pragma unroll
        for (int e = 0; e < GCH; ++e) rb[e] = (k < k_hi && jq + e < p.N) ? src[e] : T(0);
    } else {    // B[j][k]: j = tid / 4, k chunk (tid % 4) * 8
      const int j = j0 + (tid >> 2), kq = k0 + (tid & 3) * GCH;
      const T* src = p.B + (int64_t)j * p.ldb + kq;
      load_chunk<T>(src, vec, rb);
      if (!vec)
#pragma unroll
        for (int e = 0; e < GCH; ++e) rb[e] = (j < p.N && kq + e < k_hi) ? src[e] : T(0);
    }
  };
  auto stash = [&]() {
    if (!TA) {
      const int i = tid >> 2, kq = (tid & 3) * GCH;
#pragma unroll
      for (int e = 0; e < GCH; ++e) As[kq + e][i] = ra[e];
    } else {
      const int k = tid >> 3, iq = (tid & 7) * GCH;
#pragma unroll
      for (int e = 0; e < GCH; ++e) As[k][iq + e] = ra[e];
    }
    if (!TB) {
      const int k = tid >> 3, jq = (tid & 7) * GCH;
#pragma unroll
      for (int e = 0; e < GCH; ++e) Bs[k][jq + e] = rb[e];
    } else {
      const int j = tid >> 2, kq = (tid & 3) * GCH;
#pragma unroll
      for (int e = 0; e < GCH; ++e) Bs[kq + e][j] = rb[e];
    }
  };

  if (k_lo < k_hi) {
    fetch(k_lo);
    for (int k0 = k_lo; k0 < k_hi; k0 += GKT) {
      __syncthreads();
      stash();
      __syncthreads();
      if (k0 + GKT < k_hi) fetch(k0 + GKT);
#pragma unroll
      for (int kk = 0; kk < GKT / 4; ++kk) {
        const int k = kk * 4 + (lane >> 4);
        const T a0 = As[k][wr * 32 + (lane & 15)];
        const T a1 = As[k][wr * 32 + 16 + (lane & 15)];
        const T b0 = Bs[k][wc * 32 + (lane & 15)];
        const T b1 = Bs[k][wc * 32 + 16 + (lane & 15)];
        acc[0][0] = Mfma16<T>::op(a0, b0, acc[0][0]);
        acc[0][1] = Mfma16<T>::op(a0, b1, acc[0][1]);
        acc[1][0] = Mfma16<T>::op(a1, b0, acc[1][0]);
        acc[1][1] = Mfma16<T>::op(a1, b1, acc[1][1]);
      }
    }
  }

  // 16x16 block layout: col = lane % 16, row = Mfma16<T>::row(lane, e).
  if (!p.nz_flag && i0 + GT <= p.M && j0 + GT <= p.N) {
    // interior tile: the accumulate loads all in flight together, then the stores, with no
    // per-element branches (so the compiler does not wait for each store)
    T cv[2][2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = i0 + wr * 32 + a * 16 + Mfma16<T>::row(lane, e);
          const int j = j0 + wc * 32 + b * 16 + (lane & 15);
          cv[a][b][e] = (p.epi == EPI_ACCUM) ? p.Cm[(int64_t)i * p.ldc + j] : T(0);
        }
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = i0 + wr * 32 + a * 16 + Mfma16<T>::row(lane, e);
          const int j = j0 + wc * 32 + b * 16 + (lane & 15);
          T v = p.alpha * acc[a][b][e];
          if (p.row_scale) v = v * p.row_scale[p.row_bcast ? 0 : i];
          if (p.epi == EPI_ACCUM) v = cv[a][b][e] + v;
          p.Cm[(int64_t)i * p.ldc + j] = v;
        }
    return;
  }
  int nz = 0;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = i0 + wr * 32 + a * 16 + Mfma16<T>::row(lane, e);
        const int j = j0 + wc * 32 + b * 16 + (lane & 15);
        if (i < p.M && j < p.N) {
          T v = p.alpha * acc[a][b][e];
          if (p.row_scale) v = v * p.row_scale[p.row_bcast ? 0 : i];
          T* c = p.Cm + (int64_t)i * p.ldc + j;
          if (p.epi == EPI_ACCUM) v = *c + v;
          *c = v;
          nz |= (v != T(0)) || (v != v);
        }
      }
  if (p.nz_flag && nz) atomicOr(p.nz_flag, 1);
}

template <typename T, bool TA, bool TB>
__global__ __launch_bounds__(256) void k_gemm_tile(GemmArgs<T> p) {
  __shared__ T As[GKT][GT + GPad<T>::v];
  __shared__ T Bs[GKT][GT + GPad<T>::v];
  gemm_tile_body<T, TA, TB>(p, blockIdx.y, blockIdx.x, blockIdx.z, As, Bs);
}

// Two independent GEMMs in one launch: tiles [0, n1) of the flattened grid belong to p1
// (A B^T), the rest to p2 (A B); grid.z is the batch entry of both.
template <typename T>
__global__ __launch_bounds__(256) void k_gemm_pair(GemmArgs<T> p1, GemmArgs<T> p2, int n1x, int n1, int n2x) {
  __shared__ T As[GKT][GT + GPad<T>::v];
  __shared__ T Bs[GKT][GT + GPad<T>::v];
  const int b = blockIdx.x;
  if (b < n1) gemm_tile_body<T, false, true>(p1, b / n1x, b % n1x, blockIdx.z, As, Bs);
  else gemm_tile_body<T, false, false>(p2, (b - n1) / n2x, (b - n1) % n2x, blockIdx.z, As, Bs);
}

template <typename T>
inline int launch_gemm(GemmArgs<T> a, bool ta, bool tb, hipStream_t s, int batch = 1) {
  if (a.M <= 0 || a.N <= 0 || batch <= 0) return RQ_OK;
  auto al = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  auto ld_ok = [](int64_t ld) { return ((ld * (int64_t)sizeof(T)) & 15) == 0; };
  a.vec = al(a.A) && al(a.B) && ld_ok(a.lda) && ld_ok(a.ldb) && ld_ok(a.sA) && ld_ok(a.sB);
  dim3 grid((a.N + GT - 1) / GT, (a.M + GT - 1) / GT, batch), block(256);
  if (!ta && !tb) hipLaunchKernelGGL((k_gemm_tile<T, false, false>), grid, block, 0, s, a);
  else if (!ta && tb) hipLaunchKernelGGL((k_gemm_tile<T, false, true>), grid, block, 0, s, a);
  else if (ta && !tb) hipLaunchKernelGGL((k_gemm_tile<T, true, false>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((k_gemm_tile<T, true, true>), grid, block, 0, s, a);
  return hipGetLastError() == hipSuccess ? RQ_OK : RQ_EHIP;
}

// p1 = A B^T and p2 = A B (either may be empty: M or N <= 0) in one launch.
template <typename T>
inline int launch_gemm_pair(GemmArgs<T> p1, GemmArgs<T> p2, hipStream_t s, int batch = 1) {
  const bool e1 = p1.M <= 0 || p1.N <= 0, e2 = p2.M <= 0 || p2.N <= 0;
  if (batch <= 0 || (e1 && e2)) return RQ_OK;
  if (e1) return launch_gemm(p2, false, false, s, batch);
  if (e2) return launch_gemm(p1, false, true, s, batch);
  auto al = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  auto ld_ok = [](int64_t ld) { return ((ld * (int64_t)sizeof(T)) & 15) == 0; };
  p1.vec = al(p1.A) && al(p1.B) && ld_ok(p1.lda) && ld_ok(p1.ldb) && ld_ok(p1.sA) && ld_ok(p1.sB);
  p2.vec = al(p2.A) && al(p2.B) && ld_ok(p2.lda) && ld_ok(p2.ldb) && ld_ok(p2.sA) && ld_ok(p2.sB);
  const int n1x = (p1.N + GT - 1) / GT, n1 = n1x * ((p1.M + GT - 1) / GT);
  const int n2x = (p2.N + GT - 1) / GT, n2 = n2x * ((p2.M + GT - 1) / GT);
  hipLaunchKernelGGL(k_gemm_pair<T>, dim3(n1 + n2, 1, batch), dim3(256), 0, s, p1, p2, n1x, n1, n2x);
  return hipGetLastError() == hipSuccess ? RQ_OK : RQ_EHIP;
}

template <typename T>
inline GemmArgs<T> gemm_args(const T* A, int64_t lda, const T* B, int64_t ldb, T* Cm, int64_t ldc,
                             int M, int N, int K, T alpha, int epi) {
  GemmArgs<T> g{};
  g.A = A; g.lda = lda; g.B = B; g.ldb = ldb; g.Cm = Cm; g.ldc = ldc;
  g.M = M; g.N = N; g.K = K; g.alpha = alpha; g.epi = epi;
  g.krange = KR_FULL; g.lower_only = 0; g.row_scale = nullptr; g.row_bcast = 0;
  g.nz_flag = nullptr; g.skip_if_zero = nullptr; g.abort_flag = nullptr;
  g.sA = 0; g.sB = 0; g.sC = 0; g.vec = 0;
  return g;
}

}  // namespace rq
