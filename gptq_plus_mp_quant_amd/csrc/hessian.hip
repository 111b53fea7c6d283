// Saliency-weighted multi-group Hessian accumulation (GPTQPlus.add_batch,
// gptq_utils/gptq_plus_utils.py:798-857) and its finalisation (finalize_hessian, :859-908).
//
// H[g] += X^T diag(s_g) X is computed as a symmetric rank-k update: only 128x128 tiles on or
// above the diagonal are formed (the mirrored half is never computed), one workgroup per
// (tile, group).  Each workgroup streams 32-token slabs of X[:, I]
// and X[:, J] (fp16/bf16/fp32, read in place): a slab is fetched into registers as raw
// 16-byte vectors while the previous slab is multiplied, then converted to fp32 and written
// to LDS token-minor ([column][token], row stride 36 floats, so each lane reads its 8 tokens
// of one column with two conflict-free ds_read_b128).  The per-token saliency s[t, g] is folded
// into the B operand as it is written (the reference's `weighted` = fl32(x * s) is never
// materialised).  Products run on v_mfma_f32_32x32x2f32 with fp32 accumulation; each 64x64
// quarter of the tile belongs to one wave (2x2 MFMA blocks of 32x32); four workgroups share a
// CU (<= 128 VGPRs, 37 KB LDS each).  The diagonal tiles of group 0 also accumulate
// act_square = sum_t x^2, read back from the staged slab by the first 128 threads.
//
// Tail balancing: the (tile, target) items of a launch run in rounds of (CUs x 4) workgroups;
// when the last round would be partly empty, its items are split along the tokens into S
// slices (chosen so that the split work fills whole rounds).  A slice writes its partial
// tile to a caller-provided workspace; the last slice to finish (an integer counter per item)
// adds the S partials to H in slice order.  Every output element therefore still has one
// fixed summation order, and results are bitwise reproducible run to run.
#include "rq_common.h"

namespace {

constexpr int HT = 128;        // output tile edge
constexpr int HKC = 32;        // tokens per slab
constexpr int HS = HKC + 4;    // LDS row stride in floats (16-byte aligned, bank-spread)
constexpr int HTHREADS = 256;

// Raw slab fragment of one thread: 16 consecutive columns of one token, per side.
template <typename TX>
struct RawSide {
  static constexpr int NV = 16 * sizeof(TX) / 16;
  union {
    uint4 u[NV];
    TX e[16];
  };
};

__device__ __forceinline__ float to_f32(__half v) { return __half2float(v); }
__device__ __forceinline__ float to_f32(__hip_bfloat16 v) { return __bfloat162float(v); }
__device__ __forceinline__ float to_f32(float v) { return v; }

// Staging map: token k = tid & 31, column chunk = tid >> 5 (16 columns each).
template <typename TX, bool EDGE>
__device__ __forceinline__ void load_side(const TX* __restrict__ X, int64_t ntok, int64_t ldx, int C,
                                          int64_t t, int col, RawSide<TX>& r) {
  if (!EDGE) {
    if (t < ntok) {
      const uint4* q = reinterpret_cast<const uint4*>(X + t * ldx + col);
#pragma unroll
      for (int v = 0; v < RawSide<TX>::NV; ++v) r.u[v] = q[v];
    } else {
#pragma unroll
      for (int v = 0; v < RawSide<TX>::NV; ++v) r.u[v] = make_uint4(0, 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int v = 0; v < RawSide<TX>::NV; ++v) r.u[v] = make_uint4(0, 0, 0, 0);
    if (t < ntok) {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (col + e < C) r.e[e] = X[t * ldx + col + e];
    }
  }
}

// Map a linear index to an upper-triangle tile (ti <= tj) in super-row order: rows are taken
// HSR at a time and each super-row is walked column by column, so tiles that run at the same
// time on one XCD share a few I strips and a few J strips of X (L2 reuse in both operands).
constexpr int HSR = 4;
__device__ __forceinline__ void upper_tile_blocked(int t, int nt, int& ti, int& tj) {
  int r0 = 0;
  int rem = t;
  for (;;) {
    const int h = min(HSR, nt - r0);
    // tiles in this super-row: sum over tj >= r0 of min(h, tj - r0 + 1)
    const int ncol = nt - r0;
    const int cnt = (ncol >= h) ? (h * (h + 1) / 2 + (ncol - h) * h) : (ncol * (ncol + 1) / 2);
    if (rem < cnt) break;
    rem -= cnt;
    r0 += h;
  }
  const int h = min(HSR, nt - r0);
  for (int c = r0;; ++c) {
    const int k = min(h, c - r0 + 1);
    if (rem < k) {
      ti = r0 + rem;
      tj = c;
      return;
    }
    rem -= k;
  }
}

// Map a linear upper-triangle tile index to (ti, tj), ti <= tj, row-major.
__device__ __forceinline__ void upper_tile(int t, int nt, int& ti, int& tj) {
  int row = 0;
  int rem = t;
  while (rem >= nt - row) {
    rem -= nt - row;
    ++row;
  }
  ti = row;
  tj = row + rem;
}

// Partial tile of one token slice: 64 accumulator floats per thread, stored e-major so each
// store instruction of the workgroup writes 1 KB contiguously, then 128 act_square partials.
constexpr int HPART = HT * HT + HT;

template <typename TX, bool EDGE>
__device__ __forceinline__ void hessian_tile(const TX* __restrict__ X, int64_t ntok, int64_t ldx,
                                             int C, const float* __restrict__ sal, int64_t ld_sal,
                                             float* __restrict__ Hg,
                                             float* __restrict__ act_sq, int I0, int J0, bool diag,
                                             bool want_act, float (*As)[HS], float (*Bs)[HS],
                                             int64_t sbeg, int64_t send, float* __restrict__ part) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int sk = tid & 31;            // staged token
  const int sc = (tid >> 5) * 16;     // first staged column

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  float actr = 0.0f;                  // act_square partial of column I0 + tid (tid < 128)

  RawSide<TX> ra, rb;
  load_side<TX, EDGE>(X, ntok, ldx, C, sbeg * HKC + sk, I0 + sc, ra);
  if (!diag) load_side<TX, EDGE>(X, ntok, ldx, C, sbeg * HKC + sk, J0 + sc, rb);

  const int fi = lane & 31;           // fragment column within a 32-block
  const int fk = (lane >> 5) * 16;    // this lane's first token in the slab

  for (int64_t sidx = sbeg; sidx < send; ++sidx) {
    const int64_t t = sidx * HKC + sk;
    const float s = (t < ntok) ? sal[t * ld_sal] : 0.0f;
    __syncthreads();                  // previous slab fully consumed
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float xa = to_f32(ra.e[e]);
      const float xb = diag ? xa : to_f32(rb.e[e]);
      As[sc + e][sk] = xa;
      Bs[sc + e][sk] = xb * s;        // fl32(x * s): the reference's `weighted`
    }
    __syncthreads();
    if (want_act && tid < HT) {       // diagonal tiles: sum_t x^2 from the staged slab
#pragma unroll
      for (int q = 0; q < HKC; q += 4) {
        const float4 v = *reinterpret_cast<const float4*>(&As[tid][q]);
        actr += v.x * v.x;
        actr += v.y * v.y;
        actr += v.z * v.z;
        actr += v.w * v.w;
      }
    }
    if (sidx + 1 < send) {            // next slab in flight while this one is multiplied
      load_side<TX, EDGE>(X, ntok, ldx, C, t + HKC, I0 + sc, ra);
      if (!diag) load_side<TX, EDGE>(X, ntok, ldx, C, t + HKC, J0 + sc, rb);
    }
#pragma unroll
    for (int h = 0; h < 4; ++h) {     // four tokens per ds_read_b128 fragment
      const int kb = fk + h * 4;
      const float4 a0 = *reinterpret_cast<const float4*>(&As[wr * 64 + fi][kb]);
      const float4 a1 = *reinterpret_cast<const float4*>(&As[wr * 64 + 32 + fi][kb]);
      const float4 b0 = *reinterpret_cast<const float4*>(&Bs[wc * 64 + fi][kb]);
      const float4 b1 = *reinterpret_cast<const float4*>(&Bs[wc * 64 + 32 + fi][kb]);
      const float* pa0 = reinterpret_cast<const float*>(&a0);
      const float* pa1 = reinterpret_cast<const float*>(&a1);
      const float* pb0 = reinterpret_cast<const float*>(&b0);
      const float* pb1 = reinterpret_cast<const float*>(&b1);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        // MFMA step: lanes 0-31 contribute token kb+q, lanes 32-63 token 16+kb+q
        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(pa0[q], pb0[q], acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(pa0[q], pb1[q], acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(pa1[q], pb0[q], acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(pa1[q], pb1[q], acc[1][1], 0, 0, 0);
      }
    }
  }

  if (part) {
    // token slice: hand the partial tile to the workspace (summed into H by the last slice)
#pragma unroll
    for (int bi = 0; bi < 2; ++bi)
#pragma unroll
      for (int bj = 0; bj < 2; ++bj)
#pragma unroll
        for (int e = 0; e < 16; ++e) part[(bi * 32 + bj * 16 + e) * HTHREADS + tid] = acc[bi][bj][e];
    if (want_act && tid < HT) part[HT * HT + tid] = actr;
    return;
  }

  // H[g][I0 + i][J0 + j] += acc   (32x32 block layout: i = 8*(e/4) + 4*(lane/32) + e%4, j = lane%32)
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = I0 + wr * 64 + bi * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int j = J0 + wc * 64 + bj * 32 + (lane & 31);
        if (!EDGE || (i < C && j < C)) {
          float* p = Hg + (int64_t)i * C + j;
          *p = *p + acc[bi][bj][e];
        }
      }

  if (want_act && tid < HT && I0 + tid < C) act_sq[I0 + tid] += actr;
}

// One output of a launch: the Hessian of one (module, saliency group) pair.  Modules that
// read the same input (q/k/v, gate/up) are accumulated by one launch, so each X strip is
// fetched once for all of them.
constexpr int HMAXT = 32;
struct HTargets {
  const float* sal[HMAXT];   // saliency column of this target: sal[t * ld_sal]
  int64_t ld_sal[HMAXT];
  float* H[HMAXT];           // C x C output
  float* act[HMAXT];         // act_square output (one target per module) or nullptr
};

// The last slice of a split item adds the S partials (in slice order) to H and act_square.
__device__ __forceinline__ void reduce_slices(const float* __restrict__ part0, int S, float* __restrict__ Hg,
                                              float* __restrict__ act_sq, int I0, int J0, int C,
                                              bool want_act) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll 4
      for (int e = 0; e < 16; ++e) {
        const int slot = (bi * 32 + bj * 16 + e) * HTHREADS + tid;
        // partials of other workgroups: coherent (L1-bypassing) loads
        float sum = __hip_atomic_load(part0 + slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int q = 1; q < S; ++q)
          sum += __hip_atomic_load(part0 + (int64_t)q * HPART + slot, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        const int i = I0 + wr * 64 + bi * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int j = J0 + wc * 64 + bj * 32 + (lane & 31);
        if (i < C && j < C) {
          float* p = Hg + (int64_t)i * C + j;
          *p = *p + sum;
        }
      }
  if (want_act && tid < HT && I0 + tid < C) {
    float sum = __hip_atomic_load(part0 + HT * HT + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int q = 1; q < S; ++q)
      sum += __hip_atomic_load(part0 + (int64_t)q * HPART + HT * HT + tid, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    act_sq[I0 + tid] += sum;
  }
}

template <typename TX>
__global__ __launch_bounds__(HTHREADS, 4) void k_hessian_accum(
    const TX* __restrict__ X, int64_t ntok, int64_t ldx, int C, HTargets tg, int ntarg, int nt,
    int ntiles, bool vec_ok, int full, int S, float* __restrict__ ws, int* __restrict__ cnt) {
  __shared__ __attribute__((aligned(16))) float As[HT][HS];
  __shared__ __attribute__((aligned(16))) float Bs[HT][HS];
  __shared__ int last_slice;

  // Blocks [0, full) run whole items.  XCD-aware order: consecutive hardware workgroup ids
  // land on different XCDs (round robin over 8); give each XCD a contiguous run of logical
  // ids so neighbouring tiles, which share X column strips, share that XCD's L2.  Targets of
  // one tile are adjacent.  Blocks [full, full + S * (total - full)) are the token slices of
  // the remaining items, slice-minor.
  const int total = ntiles * ntarg;
  const int b = blockIdx.x;
  const int64_t nslab = (ntok + HKC - 1) / HKC;
  int logical, slice = -1;
  int64_t sbeg = 0, send = nslab;
  if (b < full) {
    const int per = full / 8, rem8 = full % 8;
    const int xcd = b % 8, idx = b / 8;
    logical = (xcd < rem8) ? xcd * (per + 1) + idx : rem8 * (per + 1) + (xcd - rem8) * per + idx;
  } else {
    const int tb = b - full;
    logical = full + tb / S;
    slice = tb % S;
    sbeg = nslab * slice / S;
    send = nslab * (slice + 1) / S;
  }
  if (logical >= total) return;
  const int g = logical % ntarg;
  int ti, tj;
  upper_tile_blocked(logical / ntarg, nt, ti, tj);
  const int I0 = ti * HT, J0 = tj * HT;
  const bool diag = (ti == tj);
  float* act_sq = tg.act[g];
  const bool want_act = diag && (act_sq != nullptr);
  float* Hg = tg.H[g];
  const bool interior = vec_ok && (J0 + HT <= C);   // I0 <= J0
  float* part0 = (slice >= 0) ? ws + (int64_t)(logical - full) * S * HPART : nullptr;
  float* part = part0 ? part0 + (int64_t)slice * HPART : nullptr;
  if (interior)
    hessian_tile<TX, false>(X, ntok, ldx, C, tg.sal[g], tg.ld_sal[g], Hg, act_sq, I0, J0, diag,
                            want_act, As, Bs, sbeg, send, part);
  else
    hessian_tile<TX, true>(X, ntok, ldx, C, tg.sal[g], tg.ld_sal[g], Hg, act_sq, I0, J0, diag,
                           want_act, As, Bs, sbeg, send, part);
  if (!part) return;
  // publish this slice, and let the last of the S slices sum them in slice order
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    int* c = cnt + (logical - full);
    const int prev = atomicAdd(c, 1);
    last_slice = (prev == S - 1);
    if (last_slice) atomicExch(c, 0);              // leave the counter zero for the next call
  }
  __syncthreads();
  if (!last_slice) return;
  __threadfence();
  reduce_slices(part0, S, Hg, act_sq, I0, J0, C, want_act);
}

}  // namespace

namespace {

// finalize_hessian (gptq_plus_utils.py:881-907): divide, symmetrise from the upper triangle,
// sanitise non-finite entries.  One 32x32 upper tile pair per workgroup.
__global__ __launch_bounds__(256) void k_hessian_finalize(float* __restrict__ H, int C, int nt,
                                                          float h_div, float sal_scale,
                                                          int apply_scale, int* nonfinite) {
  __shared__ float tile[32][33];
  __shared__ int cnt;
  const int g = blockIdx.y;
  int ti, tj;
  upper_tile(blockIdx.x, nt, ti, tj);
  float* Hg = H + (int64_t)g * C * C;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  if (threadIdx.x == 0) cnt = 0;
  for (int y = ty; y < 32; y += 8) {
    const int i = ti * 32 + y, j = tj * 32 + tx;
    float v = 0.0f;
    if (i < C && j < C) v = Hg[(int64_t)i * C + j];
    tile[y][tx] = v;
  }
  __syncthreads();
  int local = 0;
  for (int y = ty; y < 32; y += 8) {
    const int i = ti * 32 + y, j = tj * 32 + tx;
    if (i >= C || j >= C) continue;
    if (ti == tj && y > tx) continue;            // lower half of a diagonal tile: mirrored below
    float v = tile[y][tx] / h_div;
    if (apply_scale) v = v / sal_scale;
    v = 0.5f * (v + v);                           // 0.5 * (H + H^T) on the symmetric value
    if (!rq_isfinite(v)) {
      v = 0.0f;
      local += (i == j) ? 1 : 2;
    }
    Hg[(int64_t)i * C + j] = v;
    tile[y][tx] = v;
  }
  __syncthreads();
  // mirror: H[j][i] = H[i][j]; write rows of the transposed tile for coalescing
  for (int y = ty; y < 32; y += 8) {
    const int j = tj * 32 + y, i = ti * 32 + tx;   // element (j, i) takes tile[tx][y]
    if (i >= C || j >= C) continue;
    if (ti == tj && tx >= y) continue;            // diagonal tile: only strictly lower
    Hg[(int64_t)j * C + i] = tile[tx][y];
  }
  if (local) atomicAdd(&cnt, local);
  __syncthreads();
  if (threadIdx.x == 0 && cnt && nonfinite) atomicAdd(nonfinite, cnt);
}

__global__ void k_scale_vec(float* __restrict__ v, int n, float div) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) v[i] = v[i] / div;
}

}  // namespace

extern "C" int rq_version(void) { return 100; }

namespace {

// Concurrent workgroups of k_hessian_accum on the current device (CUs x occupancy).
int hessian_slots() {
  static int cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] > 0) return cache[dev];
  int cus = 0, occ = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_hessian_accum<__half>, HTHREADS, 0) !=
      hipSuccess)
    return 0;
  cache[dev] = cus * occ;
  return cache[dev];
}

// Items of the last, partly filled round and the slice count that fills rounds best
// (the finishing time of the tail in rounds is ceil(tail * S / slots) / S).
void tail_split(int64_t total, int64_t nslab, int slots, int* tail, int* S) {
  *tail = 0;
  *S = 1;
  if (slots <= 0 || total <= 0) return;
  const int64_t t = total % slots;
  if (t == 0) return;
  double best = 1.0;
  int bestS = 1;
  for (int cand = 2; cand <= 8; cand *= 2) {
    if (nslab < 4 * cand) break;                  // keep >= 4 slabs per slice
    const double rounds = (double)((t * cand + slots - 1) / slots) / cand;
    if (rounds < best - 0.05) {
      best = rounds;
      bestS = cand;
    }
  }
  if (bestS > 1) {
    *tail = (int)t;
    *S = bestS;
  }
}

// Workspace layout: one int counter per possible tail item at a fixed place (the start), so
// launches with different tails can share one workspace, then the partial tiles.
int64_t hessian_cnt_bytes(int slots) { return (((int64_t)slots * 4 + 255) / 256) * 256; }

int64_t hessian_ws_bytes(int64_t tail, int S, int slots) {
  if (tail <= 0) return 0;
  return hessian_cnt_bytes(slots) + tail * S * (int64_t)HPART * 4;
}

int launch_hessian(const void* x, int x_dtype, int64_t ntok, int64_t ldx, int C, const HTargets& tg,
                   int ntarg, void* ws, int64_t ws_bytes, hipStream_t s) {
  const int nt = (C + HT - 1) / HT;
  const int ntiles = nt * (nt + 1) / 2;
  const int64_t total = (int64_t)ntiles * ntarg;
  if (total > 0x7fffffff / 8) return RQ_EINVAL;
  const size_t esz = (x_dtype == RQ_F32) ? 4 : 2;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && (((size_t)ldx * esz) % 16 == 0);
  int tail = 0, S = 1;
  const int slots = hessian_slots();
  if (ws) tail_split(total, (ntok + HKC - 1) / HKC, slots, &tail, &S);
  const int64_t need = hessian_ws_bytes(tail, S, slots);
  if (tail > 0 && (ws_bytes < need || (reinterpret_cast<uintptr_t>(ws) & 255))) {
    tail = 0;                                     // no room: whole items only
    S = 1;
  }
  const int full = (int)(total - tail);
  int* cnt = tail > 0 ? reinterpret_cast<int*>(ws) : nullptr;
  float* wsf = tail > 0 ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + hessian_cnt_bytes(slots))
                        : nullptr;
  dim3 grid((unsigned)(full + (int64_t)tail * S)), block(HTHREADS);
  if (x_dtype == RQ_F16)
    hipLaunchKernelGGL(k_hessian_accum<__half>, grid, block, 0, s, (const __half*)x, ntok, ldx, C, tg,
                       ntarg, nt, ntiles, vec_ok, full, S, wsf, cnt);
  else if (x_dtype == RQ_BF16)
    hipLaunchKernelGGL(k_hessian_accum<__hip_bfloat16>, grid, block, 0, s, (const __hip_bfloat16*)x,
                       ntok, ldx, C, tg, ntarg, nt, ntiles, vec_ok, full, S, wsf, cnt);
  else
    hipLaunchKernelGGL(k_hessian_accum<float>, grid, block, 0, s, (const float*)x, ntok, ldx, C, tg,
                       ntarg, nt, ntiles, vec_ok, full, S, wsf, cnt);
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}

}  // namespace

extern "C" int64_t rq_hessian_workspace_bytes(int64_t ntok, int C, int ntargets) {
  if (ntok < 0 || C <= 0 || ntargets <= 0) return RQ_EINVAL;
  const int nt = (C + HT - 1) / HT;
  int64_t need = 0;
  for (int t0 = 0; t0 < ntargets; t0 += HMAXT) {   // per launch of at most 32 targets
    const int n = (ntargets - t0 < HMAXT) ? (ntargets - t0) : HMAXT;
    int tail = 0, S = 1;
    const int slots = hessian_slots();
    tail_split((int64_t)nt * (nt + 1) / 2 * n, (ntok + HKC - 1) / HKC, slots, &tail, &S);
    const int64_t b = hessian_ws_bytes(tail, S, slots);
    if (b > need) need = b;
  }
  return need;
}

extern "C" int rq_hessian_accum(const void* x, int x_dtype, int64_t ntok, int64_t ldx, int C,
                                const float* sal, int64_t ld_sal, int G, float* H, float* act_sq,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  if (!x || !sal || !H || C <= 0 || G <= 0 || ntok < 0 || ldx < C || ld_sal < G) return RQ_EINVAL;
  if (x_dtype != RQ_F16 && x_dtype != RQ_BF16 && x_dtype != RQ_F32) return RQ_EINVAL;
  if (ntok == 0) return RQ_OK;
  for (int g0 = 0; g0 < G; g0 += HMAXT) {     // up to 32 groups per launch
    const int n = (G - g0 < HMAXT) ? (G - g0) : HMAXT;
    HTargets tg{};
    for (int t = 0; t < n; ++t) {
      const int g = g0 + t;
      tg.sal[t] = sal + g;
      tg.ld_sal[t] = ld_sal;
      tg.H[t] = H + (int64_t)g * C * C;
      tg.act[t] = (g == 0) ? act_sq : nullptr;
    }
    const int rc = launch_hessian(x, x_dtype, ntok, ldx, C, tg, n, workspace, workspace_bytes,
                                  reinterpret_cast<hipStream_t>(stream));
    if (rc) return rc;
  }
  return RQ_OK;
}

extern "C" int rq_hessian_accum_multi(const void* x, int x_dtype, int64_t ntok, int64_t ldx, int C,
                                      int ntargets, const float* const* sal, const int64_t* ld_sal,
                                      float* const* H, float* const* act_sq, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  if (!x || !sal || !ld_sal || !H || C <= 0 || ntargets <= 0 || ntargets > HMAXT || ntok < 0 ||
      ldx < C)
    return RQ_EINVAL;
  if (x_dtype != RQ_F16 && x_dtype != RQ_BF16 && x_dtype != RQ_F32) return RQ_EINVAL;
  HTargets tg{};
  for (int t = 0; t < ntargets; ++t) {
    if (!sal[t] || !H[t] || ld_sal[t] < 1) return RQ_EINVAL;
    tg.sal[t] = sal[t];
    tg.ld_sal[t] = ld_sal[t];
    tg.H[t] = H[t];
    tg.act[t] = act_sq ? act_sq[t] : nullptr;
  }
  if (ntok == 0) return RQ_OK;
  return launch_hessian(x, x_dtype, ntok, ldx, C, tg, ntargets, workspace, workspace_bytes,
                        reinterpret_cast<hipStream_t>(stream));
}

extern "C" int rq_hessian_finalize(float* H, float* act_sq, int G, int C, double h_div,
                                   double sal_scale, double seq_len, int* nonfinite, void* stream) {
  if (!H || C <= 0 || G <= 0 || !(h_div > 0) || !(seq_len > 0)) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int nt = (C + 31) / 32;
  const int ntiles = nt * (nt + 1) / 2;
  // torch divides a float tensor by a Python scalar in float: a / (float)b (CPU kernel).
  hipLaunchKernelGGL(k_hessian_finalize, dim3(ntiles, G), dim3(256), 0, s, H, C, nt, (float)h_div,
                     (float)sal_scale, sal_scale != 1.0 ? 1 : 0, nonfinite);
  RQ_CHECK_LAUNCH();
  if (act_sq) {
    hipLaunchKernelGGL(k_scale_vec, dim3((C + 255) / 256), dim3(256), 0, s, act_sq, C, (float)seq_len);
    RQ_CHECK_LAUNCH();
  }
  return RQ_OK;
}
