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
// CU (<= 128 VGPRs, 37 KB LDS each).  act_square is reduced by its own kernels (below), in
// the order of the reference's CPU reduction.
//
// Tail balancing: the (tile, target) items of a launch run in rounds of (CUs x 4) workgroups;
// when the last round would be partly empty, its items are split along the tokens into S
// slices (chosen so that the split work fills whole rounds).  A slice writes its partial
// tile to a caller-provided workspace; the last slice to finish (an integer counter per item)
// adds the S partials to H in slice order.  Every output element therefore still has one
// fixed summation order, and results are bitwise reproducible run to run.
#include "rq_common.h"

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>
#include <utility>

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

// Super-row order of the off-diagonal upper-triangle tiles: tile rows are taken HSR at a time
// and each super-row is walked column by column, so tiles that run at the same time on one XCD
// share a few I strips and a few J strips of X (L2 reuse in both operands).
constexpr int HSR = 4;
// The t-th off-diagonal tile (ti < tj) in super-row order.
__device__ __forceinline__ void offdiag_tile(int t, int nt, int& ti, int& tj) {
  int r0 = 0;
  int rem = t;
  for (;;) {
    const int h = min(HSR, nt - r0);
    const int cnt = h * (h + 1) / 2 + (nt - r0 - h) * h - h;   // the super-row's tiles minus its h diagonal ones
    if (rem < cnt) break;
    rem -= cnt;
    r0 += h;
  }
  const int h = min(HSR, nt - r0);
  for (int c = r0;; ++c) {
    const int k = min(h, c - r0 + 1) - (c < r0 + h ? 1 : 0);
    if (rem < k) {
      ti = r0 + rem;
      tj = c;
      return;
    }
    rem -= k;
  }
}

// Item order of the Hessian kernels.  The item list holds every off-diagonal tile (in
// super-row order) before every diagonal tile, the
// targets of a tile consecutive.  The whole items (blocks b < full; block b runs on XCD b % 8)
// are dealt to the 8 XCDs as contiguous runs of that list, each XCD taking its proportional share
// of the off-diagonal items first and of the diagonal ones after.  The items that run side by side
// on an XCD then do equal work per step (a diagonal tile computes only its upper half), so the
// targets of a tile, which read the same X strips, start together and stay in step, and share
// those strips through the XCD's L2.  The tail's token-slice items are the list's last items
// (position = logical index).  Returns the list position of whole-item block b.
__device__ __forceinline__ int item_position(int b, int full, int od_items) {
  const int per = full / 8, rem8 = full % 8;
  const int x = b % 8, idx = b / 8;
  const int64_t len0 = (int64_t)x * per + min(x, rem8);        // whole items of the XCDs before x
  const int64_t len1 = len0 + per + (x < rem8 ? 1 : 0);
  const int64_t od_full = min((int64_t)od_items, (int64_t)full);
  const int64_t od0 = od_full * len0 / full, od1 = od_full * len1 / full;
  if (idx < od1 - od0) return (int)(od0 + idx);
  return (int)(od_full + (len0 - od0) + (idx - (od1 - od0)));
}

// Target and tile of list position pos.
__device__ __forceinline__ void item_tile(int pos, int ntarg, int nt, int& g, int& ti, int& tj) {
  const int od_items = nt * (nt - 1) / 2 * ntarg;
  if (pos < od_items) {
    g = pos % ntarg;
    offdiag_tile(pos / ntarg, nt, ti, tj);
  } else {
    const int p2 = pos - od_items;
    g = p2 % ntarg;
    ti = tj = p2 / ntarg;
  }
}



// Partial tile of one token slice: 64 accumulator floats per thread, stored e-major so each
// store instruction of the workgroup writes 1 KB contiguously.
constexpr int HPART = HT * HT;

template <typename TX, bool EDGE>
__device__ __forceinline__ void hessian_tile(const TX* __restrict__ X, int64_t ntok, int64_t ldx,
                                             int C, const float* __restrict__ sal, int64_t ld_sal,
                                             float* __restrict__ Hg, int I0, int J0, bool diag,
                                             float (*As)[HS], float (*Bs)[HS],
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

// The last slice of a split item adds the S partials (in slice order) to H.
__device__ __forceinline__ void reduce_slices(const float* __restrict__ part0, int S, float* __restrict__ Hg,
                                              int I0, int J0, int C) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  // partials of other workgroups: coherent loads, the S (<= 8) of 4 outputs issued together
  // (within this kernel's register budget), then added in slice order
#pragma unroll 1
  for (int blk = 0; blk < 16; ++blk) {
      const int bi = blk >> 3, bj = (blk >> 2) & 1, e0 = 4 * (blk & 3);
      float v[4][8];
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int q = 0; q < 8; ++q)
          v[e][q] = (q < S) ? __hip_atomic_load(part0 + (int64_t)q * HPART + (bi * 32 + bj * 16 + e0 + e) * HTHREADS + tid,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                            : 0.0f;
#pragma unroll
      for (int ee = 0; ee < 4; ++ee) {
        const int e = e0 + ee;
        float sum = v[ee][0];
#pragma unroll
        for (int q = 1; q < 8; ++q)
          if (q < S) sum += v[ee][q];
        const int i = I0 + wr * 64 + bi * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int j = J0 + wc * 64 + bj * 32 + (lane & 31);
        if (i < C && j < C) {
          float* p = Hg + (int64_t)i * C + j;
          *p = *p + sum;
        }
      }
    }
}

// Four workgroups per CU for 16-bit X; three for fp32 X, whose twice larger prefetch registers
// would otherwise spill at the four-workgroup budget of 128 VGPRs.
template <typename TX>
constexpr int accum_wgs() { return sizeof(TX) == 4 ? 3 : 4; }

template <typename TX>
__global__ __launch_bounds__(HTHREADS, accum_wgs<TX>()) void k_hessian_accum(
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
    logical = item_position(b, full, nt * (nt - 1) / 2 * ntarg);
  } else {
    const int tb = b - full;
    logical = full + tb / S;
    slice = tb % S;
    sbeg = nslab * slice / S;
    send = nslab * (slice + 1) / S;
  }
  if (logical >= total) return;
  int g, ti, tj;
  item_tile(logical, ntarg, nt, g, ti, tj);
  const int I0 = ti * HT, J0 = tj * HT;
  const bool diag = (ti == tj);
  float* Hg = tg.H[g];
  const bool interior = vec_ok && (J0 + HT <= C);   // I0 <= J0
  float* part0 = (slice >= 0) ? ws + (int64_t)(logical - full) * S * HPART : nullptr;
  float* part = part0 ? part0 + (int64_t)slice * HPART : nullptr;
  if (interior)
    hessian_tile<TX, false>(X, ntok, ldx, C, tg.sal[g], tg.ld_sal[g], Hg, I0, J0, diag, As, Bs, sbeg,
                            send, part);
  else
    hessian_tile<TX, true>(X, ntok, ldx, C, tg.sal[g], tg.ld_sal[g], Hg, I0, J0, diag, As, Bs, sbeg,
                           send, part);
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
  reduce_slices(part0, S, Hg, I0, J0, C);
}

// ---------------------------------------------------------------------------------------------
// Split-operand kernel for 16-bit inputs (the default for fp16 / bf16 X).
//
// H_ij = sum_t x_ti * w_tj with w = fl32(x * s), the reference's `weighted`.  x is exact in
// the input's 16-bit type.  w is multiplied by 2^e (one exponent per target and column,
// exact) and written as the sum of PC 16-bit pieces, p0 = rn(w), p1 = rn(w - p0),
// p2 = rn(w - p0 - p1) (round to nearest in the 16-bit type).  Each product x * p_k (11 x 11
// or 8 x 8 bits) is exact in fp32, and PC v_mfma_f32_32x32x16_{f16,bf16} per 16 tokens add
// them into fp32 accumulators.
//  * bf16, and fp16 with RQ_HMATH_SPLIT16X3 (the default): three pieces, 8 + 8 + 8 or
//    11 + 11 + 2 significant bits, cover w's 24: the reference's fp32 products, exactly.
//  * fp16 with RQ_HMATH_SPLIT16 (opt-in): two pieces carry 22 of w's 24 bits; the dropped
//    residual is at most half an ulp of p1, 2^-23 relative to w (the unit roundoff of fp32 is
//    2^-24), so each product is the reference's up to 2^-23 relative, for two thirds of the
//    MFMA work of three pieces.
// The exponent e (k_xfinish) puts the column's largest |w| in [2^14, 2^15): p0 cannot
// overflow fp16, and fp16 pieces are normal numbers for every |w| * 2^e >= 2^-1 (down to 2^-15
// of the column's largest entry); below that p1's subnormal spacing bounds the residual by
// 2^-25 * 2^-e, 2^-40 of the column's largest |w|.  bf16 pieces have fp32's exponent range;
// the same scaling is applied, harmlessly.  The epilogue multiplies the tile by 2^-e (exact)
// before adding it to H.
//
// Operands.  A pre-pass (k_xprep) writes the chunk in a fragment-blocked layout: for each
// block of 32 columns and each 16-token step, one contiguous 1 KB holding exactly the
// v_mfma_f32_32x32x16 operand of a wave (lane L = r + 32 h: tokens 8h..8h+7 of column r, zero
// padded past ntok and C), so that every operand load of the product kernel reads whole cache
// lines.  It also writes each target's saliency as a contiguous zero-padded vector and reduces
// act_square and the per-column / per-target maxima.  A workgroup (8 waves, two per SIMD, one
// workgroup per CU) owns a 256 x 256 tile of the upper triangle; wave w owns columns
// 32w..32w+31 against all 256 rows (8 blocks of 32 x 32: 128 accumulators per lane, so two
// waves fit a SIMD and the hardware interleaves one wave's loads and split with the other's
// MFMAs).  Operands are staged into a ring of LDS stages by direct global->LDS loads (wave w
// fetches row fragment w and its own column fragment, wave 0 the step's saliencies); per 16
// tokens a wave reads 8 row fragments, splits its column fragment in registers and issues
// PC x 8 MFMAs.
constexpr int XT = 256;          // workgroup tile edge
constexpr int XNPMAX = 3;        // most pieces of the weighted operand
constexpr int XWAVES = 8;        // waves per workgroup, two per SIMD
constexpr int XTHREADS = 64 * XWAVES;
constexpr int XPART = XT * XT;   // floats of one partial tile
constexpr int XTOK = 256;        // token padding of the transposed chunk / pre-pass block

template <typename TX>
struct XType;
template <>
struct XType<__half> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  typedef _Float16 v2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ floatx16 mfma(v8 a, v8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float lo(uint32_t u) { return (float)__builtin_bit_cast(v2, u).x; }
  static __device__ __forceinline__ float hi(uint32_t u) { return (float)__builtin_bit_cast(v2, u).y; }
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    v2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};
template <>
struct XType<__hip_bfloat16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  typedef __bf16 v2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ floatx16 mfma(v8 a, v8 b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float lo(uint32_t u) { return __uint_as_float(u << 16); }
  static __device__ __forceinline__ float hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    v2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
};

// One token pair of one column (x of tokens t, t+1 packed in xw): w = fl32(x * s) * 2^e for
// both, split into PC packed pieces.  fp16: each residual w - p is one v_fma_mix_f32
// (-p as an fp16 operand, times 1, plus w: exact), written out because the compiler emits a
// conversion and a subtraction for it.
template <typename TX, int PC>
__device__ __forceinline__ void split_pair(uint32_t xw, float s0, float s1, float sc, uint32_t& o0, uint32_t& o1,
                                           uint32_t& o2) {
  typedef XType<TX> T;
  float a = __builtin_fmaf(T::lo(xw), s0, 0.0f) * sc;
  float b = __builtin_fmaf(T::hi(xw), s1, 0.0f) * sc;
  if constexpr (std::is_same<TX, __half>::value && PC == 2) {
    asm("v_cvt_pk_f16_f32 %0, %2, %3\n\t"
        "v_fma_mix_f32 %2, -%0, 1.0, %2 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mix_f32 %3, -%0, 1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_cvt_pk_f16_f32 %1, %2, %3"
        : "=&v"(o0), "=&v"(o1), "+v"(a), "+v"(b));
    o2 = 0u;
  } else if constexpr (std::is_same<TX, __half>::value) {
    asm("v_cvt_pk_f16_f32 %0, %3, %4\n\t"
        "v_fma_mix_f32 %3, -%0, 1.0, %3 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mix_f32 %4, -%0, 1.0, %4 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_cvt_pk_f16_f32 %1, %3, %4\n\t"
        "v_fma_mix_f32 %3, -%1, 1.0, %3 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mix_f32 %4, -%1, 1.0, %4 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_cvt_pk_f16_f32 %2, %3, %4"
        : "=&v"(o0), "=&v"(o1), "=&v"(o2), "+v"(a), "+v"(b));
  } else {
    static_assert(PC == 3, "bf16 pieces: three");
    o0 = T::pack(a, b);
    a = a - T::lo(o0);
    b = b - T::hi(o0);
    o1 = T::pack(a, b);
    a = a - T::lo(o1);
    b = b - T::hi(o1);
    o2 = T::pack(a, b);
  }
}

template <typename TX, int PC>
__device__ __forceinline__ void split8(uint4 x, float4 s0, float4 s1, float sc, uint4 (&p)[PC]) {
  typedef XType<TX> T;
  const float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
  uint32_t o[PC][4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    float a = __builtin_fmaf(T::lo(xw[m]), s[2 * m], 0.0f);
    float b = __builtin_fmaf(T::hi(xw[m]), s[2 * m + 1], 0.0f);
    a = a * sc;
    b = b * sc;
#pragma unroll
    for (int k = 0; k < PC; ++k) {
      const uint32_t u = T::pack(a, b);
      o[k][m] = u;
      if (k + 1 < PC) {
        a = __builtin_fmaf(-T::lo(u), 1.0f, a);
        b = __builtin_fmaf(-T::hi(u), 1.0f, b);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < PC; ++k) p[k] = make_uint4(o[k][0], o[k][1], o[k][2], o[k][3]);
}

// LDS ring: XDEPTH stages (separate arrays) of one 16-token step each.  A stage holds the
// workgroup's 8 row fragments (wave w fetches fragment w), each wave's column fragment, and the
// step's 16 saliencies (wave 0, lanes 0-3); every fragment is 64 lanes x 16 B placed by lane,
// so a lane reads back exactly its own MFMA operand.  Step k of a tile (or token slice)
// starting at kbeg lives in stage (k - kbeg) % XDEPTH; the loop is unrolled by XDEPTH so that
// every stage index is a compile-time constant: the LDS reads are ordinary loads (the compiler
// places their lgkmcnt waits), and alias analysis can tell the staging writes in flight to
// other stages from the stage being read.
constexpr int XDEPTH = 8;   // 8 stages (133 KB of LDS, one workgroup per CU): 2 % faster than 4 at cfg3
constexpr int XA_BYTES = 8 * 1024;                  // row fragments of a stage
constexpr int XB_OFF = XA_BYTES;                    // column fragment of wave w at XB_OFF + 1024 w
constexpr int XS_OFF = XB_OFF + XWAVES * 1024;      // the step's 16 saliencies (64 B)
constexpr int XSTAGE = XS_OFF + 256;

struct XStages {
  uint8_t* s[XDEPTH];
};

// s_waitcnt with only the vector-memory counter limited (gfx9 encoding).
#define XWAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

__device__ __forceinline__ void lds_dma16(const void* g, uint8_t* l) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)l, 16, 0, 0);
}

// Stage step k into `st`: row fragment w and this wave's column fragment (each one contiguous
// 1 KB of the fragment-blocked chunk), and -- wave 0, lanes 0-3 -- the step's 16 saliencies.
// 2 staging loads per wave and step (wave 0: 3).
__device__ __forceinline__ void stage_step(uint8_t* st, const uint16_t* pa, const uint16_t* pb, const float* sg,
                                           int wave, int lane, int64_t k) {
  asm volatile("" : "+s"(k));
  const int64_t off = k * 512;                      // 1 KB per step and fragment
  lds_dma16(pa + off, st + wave * 1024);
  lds_dma16(pb + off, st + XB_OFF + wave * 1024);
  if (wave == 0 && lane < 4) lds_dma16(sg + 16 * k + 4 * lane, st + XS_OFF);
}

// This wave's column fragment and the saliencies of a staged step, split into pieces.
template <typename TX, int PC>
__device__ __forceinline__ void split_staged(const uint8_t* st, int wave, int lane, float sc, uint4 (&p)[PC]) {
  const uint8_t* w = static_cast<const uint8_t*>(__builtin_assume_aligned(st + XB_OFF + wave * 1024 + lane * 16, 16));
  const uint8_t* sp = static_cast<const uint8_t*>(__builtin_assume_aligned(st + XS_OFF + 32 * (lane >> 5), 16));
  split8<TX, PC>(*reinterpret_cast<const uint4*>(w), *reinterpret_cast<const float4*>(sp),
             *reinterpret_cast<const float4*>(sp + 16), sc, p);
}

// One 16-token step k of a wave.  KP = (k - kbeg) % 2 selects the register buffers (row
// fragments a and pieces p of step k, both read or made during step k-1); CUR, NXT, FILL are
// the stages of steps k, k+1 and k+XDEPTH-1.  Every wave's staging of steps k and k+1 was
// issued XDEPTH-1 and XDEPTH-2 steps ago and is followed by at least the 2 staging loads of
// each of the XDEPTH-3 steps since, so vmcnt(2 * (XDEPTH - 3)) covers this wave's part of both
// whatever the issue order within a step, and after the barrier the other waves' parts are in
// LDS too.  The barrier also orders every read of the FILL stage (the stage of step k-1, read
// during step k-2) before its refill.  RQ_STAGE_BARRIER, not __syncthreads, whose fence would
// wait for every staging load in flight.
// After the barrier: stage step k+XDEPTH-1 (row fragment w, this wave's column fragment), read
// the next step's column fragment and saliencies, then work through the row blocks in pairs:
// the pair's PC x 2 MFMAs (smallest piece first into each accumulator, the two accumulators
// alternating), with the pair's row fragments of the next step (which this step no longer
// reads) issued after its first two MFMAs and the split of one token pair of the next step's
// column fragment after the next two.  Each piece of work is pinned between sched_barriers:
// left alone, the compiler sinks all the next step's LDS reads behind the last MFMA, so every
// wave then waits on a burst of LDS reads right before the barrier (measured: MFMA busy
// 67 / 72 % -> 71 / 76 % at C = 4096 / 14336 with the reads spread after each pair's six
// MFMAs; placing them after its first two instead, and the split after the next two, gained
// another 1-1.5 % over that; groups of 4 or 8 row blocks lost 2 / 7 %).  The saliency
// staging (wave 0, lanes 0-3, a branch) comes last, so the step's main work is one scheduling
// region.  Its vmcnt accounting is unchanged: wave 0's saliency load of step k+XDEPTH-1 still
// follows that step's row / column loads.
// DIAG (a diagonal tile): row blocks below this wave's column block hold only the discarded
// lower triangle, so their row fragments are not read and their MFMAs not issued (bi < lim).
template <typename TX, int PC, bool DIAG, int KP, int CUR, int NXT, int FILL>
__device__ __forceinline__ void split_step(uint4 (&p)[2][PC], uint4 (&a)[2][8], floatx16 (&acc)[8],
                                           const XStages& L, const uint16_t* pa, const uint16_t* pb,
                                           const float* sg, float sc, int wave, int lane, int64_t k,
                                           int64_t last, int lim) {
  typedef XType<TX> T;
  typedef typename T::v8 v8;
  constexpr int NP = 1 - KP;
  XWAIT_VM(2 * (XDEPTH - 3));
  RQ_STAGE_BARRIER();
  const int64_t kf = min(k + XDEPTH - 1, last);
  {
    int64_t kk = kf;
    asm volatile("" : "+s"(kk));
    const int64_t off = kk * 512;                     // 1 KB per step and fragment
    lds_dma16(pa + off, L.s[FILL] + wave * 1024);
    lds_dma16(pb + off, L.s[FILL] + XB_OFF + wave * 1024);
  }
  const uint8_t* nxt = static_cast<const uint8_t*>(__builtin_assume_aligned(L.s[NXT] + lane * 16, 16));
  const uint8_t* w = static_cast<const uint8_t*>(
      __builtin_assume_aligned(L.s[NXT] + XB_OFF + wave * 1024 + lane * 16, 16));
  const uint8_t* sp = static_cast<const uint8_t*>(__builtin_assume_aligned(L.s[NXT] + XS_OFF + 32 * (lane >> 5), 16));
  const uint4 b = *reinterpret_cast<const uint4*>(w);
  const float4 s0 = *reinterpret_cast<const float4*>(sp);
  const float4 s1 = *reinterpret_cast<const float4*>(sp + 16);
  const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  const uint32_t xw[4] = {b.x, b.y, b.z, b.w};
  uint32_t o[XNPMAX][4];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int b0 = 2 * j, b1 = 2 * j + 1;
#pragma unroll
    for (int q = PC - 1; q >= 0; --q) {
      if (!DIAG || b0 < lim)
        acc[b0] = T::mfma(__builtin_bit_cast(v8, a[KP][b0]), __builtin_bit_cast(v8, p[KP][q]), acc[b0]);
      if (!DIAG || b1 < lim)
        acc[b1] = T::mfma(__builtin_bit_cast(v8, a[KP][b1]), __builtin_bit_cast(v8, p[KP][q]), acc[b1]);
      __builtin_amdgcn_sched_barrier(0);
      if (q == PC - 1) {            // after the first MFMA pair: the pair's next-step row fragments
        if (!DIAG || b0 < lim) a[NP][b0] = *reinterpret_cast<const uint4*>(nxt + b0 * 1024);
        if (!DIAG || b1 < lim) a[NP][b1] = *reinterpret_cast<const uint4*>(nxt + b1 * 1024);
      }
      if (q == PC - 2)              // after the second: the split of token pair j
        split_pair<TX, PC>(xw[j], sv[2 * j], sv[2 * j + 1], sc, o[0][j], o[1][j], o[2][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int q = 0; q < PC; ++q) p[NP][q] = make_uint4(o[q][0], o[q][1], o[q][2], o[q][3]);
  if (wave == 0 && lane < 4) lds_dma16(sg + 16 * kf + 4 * lane, L.s[FILL] + XS_OFF);
}

// Steps k .. k+nsteps-1 (nsteps <= XDEPTH) of the unrolled schedule: step k+J uses stage J,
// reads stage J+1 and refills stage J-1 (mod XDEPTH), and register buffer J % 2.
template <typename TX, int PC, bool DIAG, int... J>
__device__ __forceinline__ void split_round(uint4 (&p)[2][PC], uint4 (&a)[2][8], floatx16 (&acc)[8],
                                            const XStages& L, const uint16_t* pa, const uint16_t* pb,
                                            const float* sg, float sc, int wave, int lane, int64_t k,
                                            int64_t last, int lim, int nsteps, std::integer_sequence<int, J...>) {
  ((J < nsteps ? split_step<TX, PC, DIAG, J % 2, J, (J + 1) % XDEPTH, (J + XDEPTH - 1) % XDEPTH>(
                     p, a, acc, L, pa, pb, sg, sc, wave, lane, k + J, last, lim)
               : void()),
   ...);
}

// Column block of wave w: w for w < 4, 11 - w above, so the two waves that share a SIMD
// (w and w + 4) own blocks c and 7 - c: on a diagonal tile, where wave w needs only the row
// blocks up to its own, each SIMD then has 9 of the 16 blocks.
__device__ __forceinline__ int split_colblock(int wave) { return wave < 4 ? wave : 11 - wave; }

template <typename TX, int PC, bool DIAG>
__device__ __forceinline__ void split_tile(const uint16_t* __restrict__ XB, int64_t nks, int C,
                                           const float* __restrict__ sg, const float* __restrict__ scl,
                                           float* __restrict__ Hg, int R0, int C0, int64_t kbeg,
                                           int64_t kend, float* __restrict__ part, const XStages& L) {
  typedef typename XType<TX>::v8 v8;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform (an SGPR), so the DIAG row-block limit is a scalar branch: an MFMA under a
  // zero exec mask would still update its accumulators
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fh = lane >> 5;
  const int cbw = split_colblock(wave);
  const int Cw = C0 + 32 * cbw;
  const int lim = DIAG ? cbw + 1 : 8;   // row blocks this wave computes
  const int ncb = (C + 31) / 32;

  // Fragment sources in the fragment-blocked chunk: block cb of 32 columns, step k at
  // ((cb * nks + k) * 64 + lane) * 8 halves.  Blocks past the last read the last one (zero
  // padded past C); their products are discarded.
  const uint16_t* pa = XB + ((int64_t)min(R0 / 32 + wave, ncb - 1) * nks * 64 + lane) * 8;
  const uint16_t* pb = XB + ((int64_t)min(Cw / 32, ncb - 1) * nks * 64 + lane) * 8;
  const float sc = scl[min(Cw + fr, C - 1)];

  floatx16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;

  // Prologue: stage steps kbeg .. kbeg+XDEPTH-2 into stages 0 .. XDEPTH-2 and split the column
  // fragment of kbeg.  Steps past the end re-read the last one; their values are never used.
  const int64_t last = kend - 1;
#pragma unroll
  for (int h = 0; h < XDEPTH - 1; ++h) stage_step(L.s[h], pa, pb, sg, wave, lane, min(kbeg + h, last));
  uint4 p[2][PC], a[2][8];
  XWAIT_VM(2 * (XDEPTH - 2));         // this wave's staging of step kbeg
  RQ_STAGE_BARRIER();       // and the other waves'
  split_staged<TX, PC>(L.s[0], wave, lane, sc, p[0]);
  {
    const uint8_t* cur = static_cast<const uint8_t*>(__builtin_assume_aligned(L.s[0] + lane * 16, 16));
#pragma unroll
    for (int bi = 0; bi < 8; ++bi)
      if (!DIAG || bi < lim) a[0][bi] = *reinterpret_cast<const uint4*>(cur + bi * 1024);
  }

  const int64_t n = kend - kbeg;
  int64_t k = kbeg;
  static_assert(XDEPTH % 2 == 0, "register buffers alternate by step");
  constexpr auto round = std::make_integer_sequence<int, XDEPTH>();
  for (; k + XDEPTH <= kend; k += XDEPTH)
    split_round<TX, PC, DIAG>(p, a, acc, L, pa, pb, sg, sc, wave, lane, k, last, lim, XDEPTH, round);
  split_round<TX, PC, DIAG>(p, a, acc, L, pa, pb, sg, sc, wave, lane, k, last, lim, (int)(n % XDEPTH), round);
  XWAIT_VM(0);                        // no staging left in flight when the workgroup moves on

  if (part) {
    // token slice: hand the (still scaled) partial tile to the workspace (zeros for the row
    // blocks a diagonal tile does not compute)
#pragma unroll
    for (int bi = 0; bi < 8; ++bi)
#pragma unroll
      for (int e = 0; e < 16; ++e) part[(bi * 16 + e) * XTHREADS + tid] = (DIAG && bi >= lim) ? 0.0f : acc[bi][e];
    return;
  }
  // H[g][i][j] += acc * 2^-e_j   (32x32 block layout: i = 8*(e/4) + 4*(lane/32) + e%4, j = lane%32)
  // The 16 loads of a block are issued together, then the 16 stores.
  const int j = Cw + fr;
  const float inv = (j < C) ? 1.0f / scl[j] : 0.0f;
#pragma unroll
  for (int bi = 0; bi < 8; ++bi) {
    if (DIAG && bi >= lim) continue;   // below the diagonal: nothing was accumulated
    float hv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int i = R0 + 32 * bi + 8 * (e >> 2) + 4 * fh + (e & 3);
      hv[e] = (i < C && j < C) ? Hg[(int64_t)i * C + j] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int i = R0 + 32 * bi + 8 * (e >> 2) + 4 * fh + (e & 3);
      if (i < C && j < C) Hg[(int64_t)i * C + j] = hv[e] + acc[bi][e] * inv;
    }
  }
}

// The last slice of a split item adds the S partials (in slice order) to H.
__device__ __forceinline__ void reduce_split_slices(const float* __restrict__ part0, int S,
                                                    float* __restrict__ Hg, const float* __restrict__ scl,
                                                    int R0, int C0, int C, const float* __restrict__ rsc = nullptr) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int fr = lane & 31, fh = lane >> 5;
  const int j = C0 + 32 * split_colblock(wave) + fr;   // the column the slices' thread held
  const float inv = (j < C) ? 1.0f / scl[j] : 0.0f;
  // per accumulator block: the S partials of its 16 outputs loaded 8 slices at a time (S
  // uniform), added in slice order
#pragma unroll 1
  for (int bi = 0; bi < 8; ++bi) {
    float sums[16];
#pragma unroll 1
    for (int q0 = 0; q0 < S; q0 += 8) {
      float v[16][8];
#pragma unroll
      for (int e = 0; e < 16; ++e)
#pragma unroll
        for (int q = 0; q < 8; ++q)
          v[e][q] = (q0 + q < S) ? __hip_atomic_load(part0 + (int64_t)(q0 + q) * XPART + (bi * 16 + e) * XTHREADS + tid,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                 : 0.0f;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float acc = q0 == 0 ? v[e][0] : sums[e] + v[e][0];
#pragma unroll
        for (int q = 1; q < 8; ++q)
          if (q0 + q < S) acc += v[e][q];
        sums[e] = acc;
      }
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float sum = sums[e];
      const int i = R0 + 32 * bi + 8 * (e >> 2) + 4 * fh + (e & 3);
      if (i < C && j < C) {
        float* ph = Hg + (int64_t)i * C + j;
        if (rsc)   // fp32 X: 2^-(ex_i + e_j), applied in fp64 (exact)
          *ph = *ph + (float)((double)sum * ((double)inv / (double)rsc[i]));
        else
          *ph = *ph + sum * inv;
      }
    }
  }
}

// One launch covers a segment of the item list: its `segn` whole items from list position seg0
// on (od_seg of them off-diagonal), dealt to the XCDs as item_position describes, followed in the
// last segment by the tail's token slices (the list's items from `full` on, S slices each).
template <typename TX, int PC>
__global__ __launch_bounds__(XTHREADS, 1) void k_hessian_split(
    const uint16_t* __restrict__ XB, int C, const float* __restrict__ sT, int64_t lds_stride,
    const float* __restrict__ scale, HTargets tg, int ntarg, int nt, int ntiles, int64_t nks, int seg0,
    int segn, int od_seg, int full, int S, float* __restrict__ ws, int* __restrict__ cnt) {
  __shared__ __attribute__((aligned(16))) uint8_t lds0[XSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds1[XSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds2[XSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds3[XSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds4[XSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds5[XSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds6[XSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds7[XSTAGE];
  __shared__ int last_slice;
  static_assert(XDEPTH == 8, "stage arrays");
  const XStages L{{lds0, lds1, lds2, lds3, lds4, lds5, lds6, lds7}};
  // Same schedule as k_hessian_accum: XCD-aware order for whole items, then the token
  // slices of the tail items.
  const int total = ntiles * ntarg;
  const int b = blockIdx.x;
  int logical, slice = -1;
  int64_t kbeg = 0, kend = nks;
  if (b < segn) {
    logical = seg0 + item_position(b, segn, od_seg);
  } else {
    const int tb = b - segn;
    logical = full + tb / S;
    slice = tb % S;
    kbeg = nks * slice / S;
    kend = nks * (slice + 1) / S;
  }
  if (logical >= total) return;
  int g, ti, tj;
  item_tile(logical, ntarg, nt, g, ti, tj);
  const int R0 = ti * XT, C0 = tj * XT;
  float* Hg = tg.H[g];
  const float* scl = scale + (int64_t)g * C;
  float* part0 = (slice >= 0) ? ws + (int64_t)(logical - full) * S * XPART : nullptr;
  float* part = part0 ? part0 + (int64_t)slice * XPART : nullptr;
  if (R0 == C0)
    split_tile<TX, PC, true>(XB, nks, C, sT + (int64_t)g * lds_stride, scl, Hg, R0, C0, kbeg, kend, part, L);
  else
    split_tile<TX, PC, false>(XB, nks, C, sT + (int64_t)g * lds_stride, scl, Hg, R0, C0, kbeg, kend, part, L);
  if (!part) return;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    int* cp = cnt + (logical - full);
    const int prev = atomicAdd(cp, 1);
    last_slice = (prev == S - 1);
    if (last_slice) atomicExch(cp, 0);
  }
  __syncthreads();
  if (!last_slice) return;
  __threadfence();
  reduce_split_slices(part0, S, Hg, scl, R0, C0, C);
}

// ---------------------------------------------------------------------------------------------
// fp32 X (k_hessian_split32, run in the opt-in RQ_HMATH_SPLIT16 mode; by default fp32 X runs on
// the fp32 MFMA kernel): the same 256 x 256 upper tiles, with x no longer exact in 16 bits.
// The row operand is x 2^ex_i written as two fp16 pieces hi + lo (22 of x's 24 bits; k_xrows32),
// the column operand w = fl32(x * s) 2^e_j is split in the kernel from the exact fp32 x (fp32
// column fragments, k_xprep32) into w0 + w1 (as the two-piece fp16 mode), and each 16-token
// step issues hi w1, hi w0 and lo w0: 3 MFMAs per product.  The terms left out (lo w1, and the
// residuals of both splits) are each below 2^-22 of |x w|, so every product is the reference's
// fp32 product within ~2^-20.5 relative, below the rounding of the fp32 sums themselves.  The
// epilogue multiplies by 2^-(ex_i + e_j) (exact).
//
// LDS stage (one 16-token step): hi row fragments [0, 8 KB), lo row fragments [8, 16 KB), the
// fp32 column fragment of wave w at 16 KB + 2 KB w (two 1 KB halves), the 16 saliencies.  A step
// runs in two phases: (A) hi x (w1, w0) while the lo rows of this step are read and the next
// step's column fragment is split; (B) lo x w0 while the next step's hi rows are read.
constexpr int X32DEPTH = 4;   // stages of 32.25 KB: 4 fit the LDS
constexpr int X3_HI = 0;
constexpr int X3_LO = 8 * 1024;
constexpr int X3_COL = 16 * 1024;
constexpr int X3_SAL = X3_COL + XWAVES * 2048;
constexpr int X3_STAGE = X3_SAL + 256;

// Stage step k: hi and lo row fragment w, this wave's fp32 column fragment (two halves), and
// -- wave 0, lanes 0-3 -- the step's 16 saliencies.  4 staging loads per wave (wave 0: 5).
__device__ __forceinline__ void stage_step32(uint8_t* st, const uint16_t* ph, const uint16_t* pl,
                                             const float* pc, const float* sg, int wave, int lane,
                                             int64_t k) {
  asm volatile("" : "+s"(k));
  lds_dma16(ph + k * 512, st + X3_HI + wave * 1024);
  lds_dma16(pl + k * 512, st + X3_LO + wave * 1024);
  lds_dma16(pc + k * 512, st + X3_COL + wave * 2048);
  lds_dma16(pc + k * 512 + 256, st + X3_COL + wave * 2048 + 1024);
  if (wave == 0 && lane < 4) lds_dma16(sg + 16 * k + 4 * lane, st + X3_SAL);
}

// w = fl32(x * s) * sc for 8 tokens (exact x), split into two packed fp16 pieces.
__device__ __forceinline__ void split8_f32(const float (&x)[8], const float (&sv)[8], float sc, uint4 (&p)[2]) {
  uint32_t o0[4], o1[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    float a = __builtin_fmaf(x[2 * m], sv[2 * m], 0.0f) * sc;
    float b = __builtin_fmaf(x[2 * m + 1], sv[2 * m + 1], 0.0f) * sc;
    asm("v_cvt_pk_f16_f32 %0, %2, %3\n\t"
        "v_fma_mix_f32 %2, -%0, 1.0, %2 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mix_f32 %3, -%0, 1.0, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_cvt_pk_f16_f32 %1, %2, %3"
        : "=&v"(o0[m]), "=&v"(o1[m]), "+v"(a), "+v"(b));
  }
  p[0] = make_uint4(o0[0], o0[1], o0[2], o0[3]);
  p[1] = make_uint4(o1[0], o1[1], o1[2], o1[3]);
}

// This wave's fp32 column fragment and the saliencies of a staged step.
__device__ __forceinline__ void read_col32(const uint8_t* st, int wave, int lane, float (&x)[8], float (&sv)[8]) {
  const uint8_t* c = st + X3_COL + wave * 2048 + lane * 16;
  const float4 a = *reinterpret_cast<const float4*>(__builtin_assume_aligned(c, 16));
  const float4 b = *reinterpret_cast<const float4*>(__builtin_assume_aligned(c + 1024, 16));
  const uint8_t* sp = st + X3_SAL + 32 * (lane >> 5);
  const float4 s0 = *reinterpret_cast<const float4*>(__builtin_assume_aligned(sp, 16));
  const float4 s1 = *reinterpret_cast<const float4*>(__builtin_assume_aligned(sp + 16, 16));
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
  sv[0] = s0.x; sv[1] = s0.y; sv[2] = s0.z; sv[3] = s0.w; sv[4] = s1.x; sv[5] = s1.y; sv[6] = s1.z; sv[7] = s1.w;
}

// One 16-token step k (stages CUR = k, NXT = k+1, FILL = k+X32DEPTH-1).  Waits as split_step:
// this step's and the next step's staging must be complete (phase A reads the lo rows of k and
// the column fragment of k+1, phase B the hi rows of k+1), so vmcnt(4 * (X32DEPTH - 3)).
template <bool DIAG, int CUR, int NXT, int FILL>
__device__ __forceinline__ void split_step32(uint4 (&p)[2], uint4 (&ah)[8], uint4 (&al)[8], floatx16 (&acc)[8],
                                             const XStages& L, const uint16_t* ph, const uint16_t* pl,
                                             const float* pc, const float* sg, float sc, int wave, int lane,
                                             int64_t k, int64_t last, int lim) {
  typedef XType<__half>::v8 v8;
  XWAIT_VM(4 * (X32DEPTH - 3));
  RQ_STAGE_BARRIER();
  stage_step32(L.s[FILL], ph, pl, pc, sg, wave, lane, min(k + X32DEPTH - 1, last));
  // phase A: hi rows x (w1, w0); the lo rows of this step and the next column fragment are read
  const uint8_t* cur = static_cast<const uint8_t*>(__builtin_assume_aligned(L.s[CUR] + X3_LO + lane * 16, 16));
#pragma unroll
  for (int bi = 0; bi < 8; ++bi)
    if (!DIAG || bi < lim) al[bi] = *reinterpret_cast<const uint4*>(cur + bi * 1024);
  float x[8], sv[8];
  read_col32(L.s[NXT], wave, lane, x, sv);
#pragma unroll
  for (int bi = 0; bi < 8; ++bi)
    if (!DIAG || bi < lim)
      acc[bi] = XType<__half>::mfma(__builtin_bit_cast(v8, ah[bi]), __builtin_bit_cast(v8, p[1]), acc[bi]);
  uint4 pn[2];
  split8_f32(x, sv, sc, pn);
#pragma unroll
  for (int bi = 0; bi < 8; ++bi)
    if (!DIAG || bi < lim)
      acc[bi] = XType<__half>::mfma(__builtin_bit_cast(v8, ah[bi]), __builtin_bit_cast(v8, p[0]), acc[bi]);
  // phase B: lo rows x w0; the next step's hi rows are read
  const uint8_t* nxt = static_cast<const uint8_t*>(__builtin_assume_aligned(L.s[NXT] + X3_HI + lane * 16, 16));
#pragma unroll
  for (int bi = 0; bi < 8; ++bi)
    if (!DIAG || bi < lim)
      acc[bi] = XType<__half>::mfma(__builtin_bit_cast(v8, al[bi]), __builtin_bit_cast(v8, p[0]), acc[bi]);
#pragma unroll
  for (int bi = 0; bi < 8; ++bi)
    if (!DIAG || bi < lim) ah[bi] = *reinterpret_cast<const uint4*>(nxt + bi * 1024);
  p[0] = pn[0];
  p[1] = pn[1];
}

template <bool DIAG, int... J>
__device__ __forceinline__ void split_round32(uint4 (&p)[2], uint4 (&ah)[8], uint4 (&al)[8], floatx16 (&acc)[8],
                                              const XStages& L, const uint16_t* ph, const uint16_t* pl,
                                              const float* pc, const float* sg, float sc, int wave, int lane,
                                              int64_t k, int64_t last, int lim, int nsteps,
                                              std::integer_sequence<int, J...>) {
  ((J < nsteps ? split_step32<DIAG, J, (J + 1) % X32DEPTH, (J + X32DEPTH - 1) % X32DEPTH>(
                     p, ah, al, acc, L, ph, pl, pc, sg, sc, wave, lane, k + J, last, lim)
               : void()),
   ...);
}

// Tile (R0, C0) of one target over steps [kbeg, kend): as split_tile, with the fp32 operands.
template <bool DIAG>
__device__ __forceinline__ void split_tile32(const uint16_t* __restrict__ XH, const uint16_t* __restrict__ XL,
                                             const float* __restrict__ XC, int64_t nks, int C,
                                             const float* __restrict__ sg, const float* __restrict__ scl,
                                             const float* __restrict__ rsc, float* __restrict__ Hg, int R0,
                                             int C0, int64_t kbeg, int64_t kend, float* __restrict__ part,
                                             const XStages& L) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 31, fh = lane >> 5;
  const int cbw = split_colblock(wave);
  const int Cw = C0 + 32 * cbw;
  const int lim = DIAG ? cbw + 1 : 8;
  const int ncb = (C + 31) / 32;
  const int64_t rb = (int64_t)min(R0 / 32 + wave, ncb - 1) * nks * 64 + lane;
  const uint16_t* ph = XH + rb * 8;
  const uint16_t* pl = XL + rb * 8;
  const float* pc = XC + ((int64_t)min(Cw / 32, ncb - 1) * nks * 128 + lane) * 4;
  const float sc = scl[min(Cw + fr, C - 1)];

  floatx16 acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;

  const int64_t last = kend - 1;
#pragma unroll
  for (int h = 0; h < X32DEPTH - 1; ++h) stage_step32(L.s[h], ph, pl, pc, sg, wave, lane, min(kbeg + h, last));
  uint4 p[2], ah[8], al[8];
  XWAIT_VM(4 * (X32DEPTH - 2));         // this wave's staging of step kbeg
  RQ_STAGE_BARRIER();       // and the other waves'
  {
    float x[8], sv[8];
    read_col32(L.s[0], wave, lane, x, sv);
    split8_f32(x, sv, sc, p);
    const uint8_t* cur = static_cast<const uint8_t*>(__builtin_assume_aligned(L.s[0] + X3_HI + lane * 16, 16));
#pragma unroll
    for (int bi = 0; bi < 8; ++bi)
      if (!DIAG || bi < lim) ah[bi] = *reinterpret_cast<const uint4*>(cur + bi * 1024);
  }
  const int64_t n = kend - kbeg;
  int64_t k = kbeg;
  constexpr auto round = std::make_integer_sequence<int, X32DEPTH>();
  for (; k + X32DEPTH <= kend; k += X32DEPTH)
    split_round32<DIAG>(p, ah, al, acc, L, ph, pl, pc, sg, sc, wave, lane, k, last, lim, X32DEPTH, round);
  split_round32<DIAG>(p, ah, al, acc, L, ph, pl, pc, sg, sc, wave, lane, k, last, lim, (int)(n % X32DEPTH), round);
  XWAIT_VM(0);

  if (part) {
#pragma unroll
    for (int bi = 0; bi < 8; ++bi)
#pragma unroll
      for (int e = 0; e < 16; ++e) part[(bi * 16 + e) * XTHREADS + tid] = (DIAG && bi >= lim) ? 0.0f : acc[bi][e];
    return;
  }
  // H[g][i][j] += acc * 2^-(ex_i + e_j), the two exact scalings applied in fp64
  const int j = Cw + fr;
  const double inv = (j < C) ? 1.0 / (double)scl[j] : 0.0;
#pragma unroll
  for (int bi = 0; bi < 8; ++bi) {
    if (DIAG && bi >= lim) continue;
    float hv[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int i = R0 + 32 * bi + 8 * (e >> 2) + 4 * fh + (e & 3);
      hv[e] = (i < C && j < C) ? Hg[(int64_t)i * C + j] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int i = R0 + 32 * bi + 8 * (e >> 2) + 4 * fh + (e & 3);
      if (i < C && j < C) Hg[(int64_t)i * C + j] = hv[e] + (float)((double)acc[bi][e] * (inv / (double)rsc[i]));
    }
  }
}

__global__ __launch_bounds__(XTHREADS, 1) void k_hessian_split32(
    const uint16_t* __restrict__ XH, const uint16_t* __restrict__ XL, const float* __restrict__ XC, int C,
    const float* __restrict__ sT, int64_t lds_stride, const float* __restrict__ scale,
    const float* __restrict__ rscale, HTargets tg, int ntarg, int nt, int ntiles, int64_t nks, int full, int S,
    float* __restrict__ ws, int* __restrict__ cnt) {
  __shared__ __attribute__((aligned(16))) uint8_t lds0[X3_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds1[X3_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds2[X3_STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds3[X3_STAGE];
  __shared__ int last_slice;
  static_assert(X32DEPTH == 4, "stage arrays");
  const XStages L{{lds0, lds1, lds2, lds3}};
  const int total = ntiles * ntarg;
  const int b = blockIdx.x;
  int logical, slice = -1;
  int64_t kbeg = 0, kend = nks;
  if (b < full) {
    logical = item_position(b, full, nt * (nt - 1) / 2 * ntarg);
  } else {
    const int tb = b - full;
    logical = full + tb / S;
    slice = tb % S;
    kbeg = nks * slice / S;
    kend = nks * (slice + 1) / S;
  }
  if (logical >= total) return;
  int g, ti, tj;
  item_tile(logical, ntarg, nt, g, ti, tj);
  const int R0 = ti * XT, C0 = tj * XT;
  float* Hg = tg.H[g];
  const float* scl = scale + (int64_t)g * C;
  float* part0 = (slice >= 0) ? ws + (int64_t)(logical - full) * S * XPART : nullptr;
  float* part = part0 ? part0 + (int64_t)slice * XPART : nullptr;
  if (R0 == C0)
    split_tile32<true>(XH, XL, XC, nks, C, sT + (int64_t)g * lds_stride, scl, rscale, Hg, R0, C0, kbeg, kend,
                       part, L);
  else
    split_tile32<false>(XH, XL, XC, nks, C, sT + (int64_t)g * lds_stride, scl, rscale, Hg, R0, C0, kbeg, kend,
                        part, L);
  if (!part) return;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    int* cp = cnt + (logical - full);
    const int prev = atomicAdd(cp, 1);
    last_slice = (prev == S - 1);
    if (last_slice) atomicExch(cp, 0);
  }
  __syncthreads();
  if (!last_slice) return;
  __threadfence();
  reduce_split_slices(part0, S, Hg, scl, R0, C0, C, rscale);
}

// Pre-pass over one 64-column x 256-token block of X: the block in the fragment-blocked
// layout read by k_hessian_split (zeros past ntok and past C), each column's max |x| and
// sum_t x^2 for this token block, and (first column block only) each target's saliency,
// contiguous and zero padded, with its max |s|.  Two tokens of one column share a 32-bit LDS word; the row stride of 129 words
// keeps the transposing writes free of bank conflicts.
constexpr int XPC = 64;            // columns per pre-pass block
constexpr int XPRS = XTOK / 2 + 1; // LDS row stride in words
template <typename TX>
__global__ __launch_bounds__(256) void k_xprep(const TX* __restrict__ X, int64_t ntok, int64_t ldx, int C,
                                               bool vec_ok, uint16_t* __restrict__ XB, int64_t nks,
                                               HTargets tg, int ntarg, float* __restrict__ sT, int64_t lds,
                                               float* __restrict__ mpart, float* __restrict__ apart,
                                               float* __restrict__ spart) {
  __shared__ uint32_t tile[XPC][XPRS];
  __shared__ unsigned smx[HMAXT];
  const int tid = threadIdx.x;
  const int c0 = blockIdx.x * XPC;
  const int ch = blockIdx.y;
  const int64_t t0 = (int64_t)ch * XTOK;
  const uint16_t* Xb = reinterpret_cast<const uint16_t*>(X);
  // load: 8 column groups (8 columns, 16 B) x 128 token pairs; lane = group + 8 * pair.  A
  // block inside the chunk (every workgroup but the edge ones) issues its 8 loads per thread
  // before using any; the edge blocks load element by element with bounds checks.
  auto put = [&](int v, uint4 q0, uint4 q1) __attribute__((always_inline)) {
    const int grp = v & 7, tp = v >> 3;
    const uint32_t a[4] = {q0.x, q0.y, q0.z, q0.w}, b[4] = {q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      tile[8 * grp + 2 * k][tp] = (a[k] & 0xffffu) | (b[k] << 16);
      tile[8 * grp + 2 * k + 1][tp] = (a[k] >> 16) | (b[k] & 0xffff0000u);
    }
  };
  if (vec_ok && c0 + XPC <= C && t0 + XTOK <= ntok) {
    uint4 q[8];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int v = tid + 256 * it;
      const int grp = v & 7, tp = v >> 3;
      const uint16_t* src = Xb + (t0 + 2 * tp) * ldx + c0 + 8 * grp;
      q[2 * it] = *reinterpret_cast<const uint4*>(src);
      q[2 * it + 1] = *reinterpret_cast<const uint4*>(src + ldx);
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) put(tid + 256 * it, q[2 * it], q[2 * it + 1]);
  } else {
#pragma unroll
    for (int v = tid; v < 8 * (XTOK / 2); v += 256) {
      const int grp = v & 7, tp = v >> 3;
      const int cb = c0 + 8 * grp;
      uint32_t e[2][8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t t = t0 + 2 * tp + h;
        if (vec_ok && cb + 8 <= C && t < ntok) {
          const uint4 q = *reinterpret_cast<const uint4*>(Xb + t * ldx + cb);
          e[h][0] = q.x & 0xffffu; e[h][1] = q.x >> 16; e[h][2] = q.y & 0xffffu; e[h][3] = q.y >> 16;
          e[h][4] = q.z & 0xffffu; e[h][5] = q.z >> 16; e[h][6] = q.w & 0xffffu; e[h][7] = q.w >> 16;
        } else {
#pragma unroll
          for (int k = 0; k < 8; ++k) e[h][k] = (t < ntok && cb + k < C) ? Xb[t * ldx + cb + k] : 0u;
        }
      }
      const uint4 q0 = make_uint4(e[0][0] | (e[0][1] << 16), e[0][2] | (e[0][3] << 16), e[0][4] | (e[0][5] << 16),
                                  e[0][6] | (e[0][7] << 16));
      const uint4 q1 = make_uint4(e[1][0] | (e[1][1] << 16), e[1][2] | (e[1][3] << 16), e[1][4] | (e[1][5] << 16),
                                  e[1][6] | (e[1][7] << 16));
      put(v, q0, q1);
    }
  }
  __syncthreads();
  // store: the block's two 32-column groups x 16 steps, fragment-major: chunk (cb, kb) is 1 KB,
  // lane L = fr + 32 fh holding tokens 16 kb + 8 fh .. +7 of column 32 cb + fr (zeros past C)
  const int ncb = (C + 31) / 32;
  for (int v = tid; v < 2 * (XTOK / 16) * 64; v += 256) {
    const int L = v & 63, kbl = (v >> 6) & (XTOK / 16 - 1), cbl = v >> 10;
    const int cb = c0 / 32 + cbl;
    if (cb < ncb) {
      const uint32_t* src = &tile[32 * cbl + (L & 31)][8 * kbl + 4 * (L >> 5)];
      *reinterpret_cast<uint4*>(XB + (((int64_t)cb * nks + (int64_t)ch * (XTOK / 16) + kbl) * 64 + L) * 8) =
          make_uint4(src[0], src[1], src[2], src[3]);
    }
  }
  // column statistics: 4 threads per column, 64 tokens each.  The 256 tokens are one level-2
  // block of the reference's CPU reduction of act_square (act_square_l2 below): each thread
  // forms its four level-1 sums (16 tokens, square then add, from zero), and one thread per
  // column adds the 16 level-1 sums in order.  Tokens past ntok are zero: they add nothing.
  {
    __shared__ float qm[4][XPC], ql1[16][XPC];
    const int cl = tid & (XPC - 1), part = tid >> 6;
    float m = 0.0f;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      float a = 0.0f;
#pragma unroll
      for (int w = part * (XTOK / 8) + 8 * b; w < part * (XTOK / 8) + 8 * b + 8; ++w) {
        const uint32_t u = tile[cl][w];
        const float v0 = XType<TX>::lo(u), v1 = XType<TX>::hi(u);
        m = fmaxf(m, fabsf(v0));
        a = a + v0 * v0;
        m = fmaxf(m, fabsf(v1));
        a = a + v1 * v1;
      }
      ql1[4 * part + b][cl] = a;
    }
    qm[part][cl] = m;
    if (tid < HMAXT) smx[tid] = 0u;
    __syncthreads();
    if (tid < XPC && c0 + tid < C) {
      mpart[(int64_t)ch * C + c0 + tid] = fmaxf(fmaxf(qm[0][tid], qm[1][tid]), fmaxf(qm[2][tid], qm[3][tid]));
      float l2 = 0.0f;
#pragma unroll
      for (int b = 0; b < 16; ++b) l2 = l2 + ql1[b][tid];
      apart[(int64_t)ch * C + c0 + tid] = l2;
    }
  }
  if (blockIdx.x != 0) return;
  for (int g = 0; g < ntarg; ++g) {
    const int64_t t = t0 + tid;
    const float s = (t < ntok) ? tg.sal[g][t * tg.ld_sal[g]] : 0.0f;
    sT[(int64_t)g * lds + t] = s;
    atomicMax(&smx[g], __float_as_uint(fabsf(s)));
  }
  __syncthreads();
  if (tid < ntarg) spart[(int64_t)ch * HMAXT + tid] = __uint_as_float(smx[tid]);
}

// Reduce the token blocks' maxima into the per (target, column) scale 2^e with e = 15 - E for
// max|x_c| * max|s_g| = f * 2^E, f in [0.5, 1).  A workgroup takes 32 columns; 8 threads per
// column each take one eighth of the blocks (maxima are exact in any order).  act_square is
// finished by k_act_finish.
constexpr int XF_COLS = 32;
constexpr int XF_SEG = 8;
__global__ __launch_bounds__(256) void k_xfinish(int C, int nchunk, int ntarg, const float* __restrict__ mpart,
                                                 const float* __restrict__ spart, float* __restrict__ scale,
                                                 float* __restrict__ rscale) {
  __shared__ float smax[XF_SEG][HMAXT];
  __shared__ float pm[XF_SEG][XF_COLS];
  const int t = threadIdx.x;
  const int lane32 = t & 31, seg = t >> 5;
  {
    float m = 0.0f;
    if (lane32 < ntarg)
      for (int ch = seg; ch < nchunk; ch += XF_SEG) m = fmaxf(m, spart[(int64_t)ch * HMAXT + lane32]);
    smax[seg][lane32] = m;
  }
  const int c = blockIdx.x * XF_COLS + lane32;
  const int ch0 = (int)((int64_t)nchunk * seg / XF_SEG), ch1 = (int)((int64_t)nchunk * (seg + 1) / XF_SEG);
  float m = 0.0f;
  if (c < C) {
#pragma unroll 8
    for (int ch = ch0; ch < ch1; ++ch) m = fmaxf(m, mpart[(int64_t)ch * C + c]);
  }
  pm[seg][lane32] = m;
  __syncthreads();
  if (seg != 0 || c >= C) return;
  float mt = pm[0][lane32];
#pragma unroll
  for (int q = 1; q < XF_SEG; ++q) mt = fmaxf(mt, pm[q][lane32]);
  if (rscale) {   // fp32 X: the column's row-piece scale 2^ex, max|x_c| * 2^ex in [2^14, 2^15)
    int ex = 0;
    if (mt > 0.0f && mt <= 3.402823466e38f) {
      int E = 0;
      (void)frexpf(mt, &E);
      ex = 15 - E;
      ex = ex < -100 ? -100 : (ex > 100 ? 100 : ex);
    }
    rscale[c] = ldexpf(1.0f, ex);
  }
  for (int g = 0; g < ntarg; ++g) {
    float sm = smax[0][g];
#pragma unroll
    for (int q = 1; q < XF_SEG; ++q) sm = fmaxf(sm, smax[q][g]);
    const float mm = mt * sm;
    int e = 0;
    if (mm > 0.0f && mm <= 3.402823466e38f) {
      int E = 0;
      (void)frexpf(mm, &E);
      e = 15 - E;
      e = e < -100 ? -100 : (e > 100 ? 100 : e);
    }
    scale[(int64_t)g * C + c] = ldexpf(1.0f, e);
  }
}

// fp32 X, pass 1 over one 64-column x 256-token block: the block as fp32 column fragments for
// k_hessian_split32 (per 32 columns and 16-token step, 2 KB: half q in {0, 1}, lane
// L = fr + 32 fh holding tokens 8 fh + 4 q .. +3 of column fr; zeros past ntok and C), each
// column's max |x| and its level-2 act_square sum for this block (as k_xprep), and (first
// column block only) the targets' saliencies.  LDS holds the block column-major, row stride 257
// floats, so that the transposing writes and the fragment reads are free of bank conflicts.
constexpr int XPRS32 = XTOK + 1;
__global__ __launch_bounds__(256) void k_xprep32(const float* __restrict__ X, int64_t ntok, int64_t ldx, int C,
                                                 bool vec_ok, float4* __restrict__ XC, int64_t nks,
                                                 HTargets tg, int ntarg, float* __restrict__ sT, int64_t lds,
                                                 float* __restrict__ mpart, float* __restrict__ apart,
                                                 float* __restrict__ spart) {
  __shared__ float tile[XPC][XPRS32];
  __shared__ unsigned smx[HMAXT];
  const int tid = threadIdx.x;
  const int c0 = blockIdx.x * XPC;
  const int ch = blockIdx.y;
  const int64_t t0 = (int64_t)ch * XTOK;
  // load: 16 float4 per token row, 16 rows per pass.  A block inside the chunk issues 8 loads
  // per thread before using any; the edge blocks check every element.
  if (vec_ok && c0 + XPC <= C && t0 + XTOK <= ntok) {
#pragma unroll
    for (int v0 = tid; v0 < 16 * XTOK; v0 += 256 * 8) {
      float4 f[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int v = v0 + 256 * u;
        f[u] = *reinterpret_cast<const float4*>(X + (t0 + (v >> 4)) * ldx + c0 + 4 * (v & 15));
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int v = v0 + 256 * u;
        const int q = v & 15, tr = v >> 4;
        tile[4 * q][tr] = f[u].x;
        tile[4 * q + 1][tr] = f[u].y;
        tile[4 * q + 2][tr] = f[u].z;
        tile[4 * q + 3][tr] = f[u].w;
      }
    }
  } else {
#pragma unroll 4
    for (int v = tid; v < 16 * XTOK; v += 256) {
      const int q = v & 15, tr = v >> 4;
      const int cb = c0 + 4 * q;
      const int64_t t = t0 + tr;
      float e[4];
      if (vec_ok && cb + 4 <= C && t < ntok) {
        const float4 f = *reinterpret_cast<const float4*>(X + t * ldx + cb);
        e[0] = f.x; e[1] = f.y; e[2] = f.z; e[3] = f.w;
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) e[k] = (t < ntok && cb + k < C) ? X[t * ldx + cb + k] : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) tile[4 * q + k][tr] = e[k];
    }
  }
  __syncthreads();
  const int ncb = (C + 31) / 32;
  for (int v = tid; v < 2 * (XTOK / 16) * 2 * 64; v += 256) {
    const int L = v & 63, q = (v >> 6) & 1, kbl = (v >> 7) & (XTOK / 16 - 1), cbl = v >> 11;
    const int cb = c0 / 32 + cbl;
    if (cb < ncb) {
      const float* src = &tile[32 * cbl + (L & 31)][16 * kbl + 8 * (L >> 5) + 4 * q];
      XC[(((int64_t)cb * nks + (int64_t)ch * (XTOK / 16) + kbl) * 2 + q) * 64 + L] =
          make_float4(src[0], src[1], src[2], src[3]);
    }
  }
  {
    __shared__ float qm[4][XPC], ql1[16][XPC];
    const int cl = tid & (XPC - 1), part = tid >> 6;
    float m = 0.0f;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      float a = 0.0f;
#pragma unroll
      for (int w = part * (XTOK / 4) + 16 * b; w < part * (XTOK / 4) + 16 * b + 16; ++w) {
        const float v0 = tile[cl][w];
        m = fmaxf(m, fabsf(v0));
        a = a + v0 * v0;
      }
      ql1[4 * part + b][cl] = a;
    }
    qm[part][cl] = m;
    if (tid < HMAXT) smx[tid] = 0u;
    __syncthreads();
    if (tid < XPC && c0 + tid < C) {
      mpart[(int64_t)ch * C + c0 + tid] = fmaxf(fmaxf(qm[0][tid], qm[1][tid]), fmaxf(qm[2][tid], qm[3][tid]));
      float l2 = 0.0f;
#pragma unroll
      for (int b = 0; b < 16; ++b) l2 = l2 + ql1[b][tid];
      apart[(int64_t)ch * C + c0 + tid] = l2;
    }
  }
  if (blockIdx.x != 0) return;
  for (int g = 0; g < ntarg; ++g) {
    const int64_t t = t0 + tid;
    const float s = (t < ntok) ? tg.sal[g][t * tg.ld_sal[g]] : 0.0f;
    sT[(int64_t)g * lds + t] = s;
    atomicMax(&smx[g], __float_as_uint(fabsf(s)));
  }
  __syncthreads();
  if (tid < ntarg) spart[(int64_t)ch * HMAXT + tid] = __uint_as_float(smx[tid]);
}

// fp32 X, pass 2: the row pieces of every fragment, hi = rn16(x 2^ex) and lo = rn16(x 2^ex - hi)
// (fp16, x 2^ex - hi exact in fp32), in the layout of k_xprep's fragments; 2^ex = rscale[c].
__global__ __launch_bounds__(256) void k_xrows32(const float4* __restrict__ XC, int64_t nfrag, int C, int64_t nks,
                                                 const float* __restrict__ rscale, uint4* __restrict__ XH,
                                                 uint4* __restrict__ XL) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;   // (fragment, lane)
  if (v >= nfrag * 64) return;
  const int L = (int)(v & 63);
  const int64_t f = v >> 6;
  const int c = (int)(f / nks) * 32 + (L & 31);
  const float rs = (c < C) ? rscale[c] : 1.0f;
  const float4 a = XC[(f * 2) * 64 + L], b = XC[(f * 2 + 1) * 64 + L];
  const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const float u0 = x[2 * m] * rs, u1 = x[2 * m + 1] * rs;
    const h2 ph = {(_Float16)u0, (_Float16)u1};
    const h2 pl = {(_Float16)(u0 - (float)ph.x), (_Float16)(u1 - (float)ph.y)};
    hi[m] = __builtin_bit_cast(uint32_t, ph);
    lo[m] = __builtin_bit_cast(uint32_t, pl);
  }
  XH[v] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  XL[v] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
}

// ---------------------------------------------------------------------------------------------
// act_square += sum_t x_t^2 of one add_batch call (gptq_plus_utils.py:856:
// `self.act_square.add_((inp ** 2).sum(0))` on the fp32 chunk), summed in the order of the
// CPU reduction that line runs, so that act_order's argsort (:1046) sees the reference's values
// bit for bit (near ties would otherwise swap columns).  That reduction (ATen's cascade sum of
// a row-major [n, C] fp32 tensor over its rows) forms each column's sum over a sequence of
// `count` elements in four levels.  With p = max(4, ceil(log2 count) / 4) and step = 2^p:
// level 1 adds `step` consecutive elements from zero, level 2 adds `step` level-1 sums from
// zero, level 3 adds `step` level-2 sums from zero, and level 4 adds every complete level-3
// sum in order.  The partial sums an incomplete block leaves at levels 1-3 (a1, a2, a3) and
// the level-4 sum a4 give ((a1 + a2) + a3) + a4.  Columns [0, 32 floor(C / 32)) (ATen's
// four-vector inner loop) are one sequence of the n rows each.  The other columns are reduced
// as four interleaved sequences, rows m, m + 4, m + 8, ... (n / 4 elements each, m < 4), the
// n mod 4 leftover rows added to the first, then ((s0 + s1) + s2) + s3.  (For C mod 32 in
// [4, 8) ATen reduces the first four of those columns either way, depending on n.)
//
// Work is split over "virtual columns": v = c for the first region (one lane), and
// v = 4 (c - c_lo) + m for the interleaved region (four lanes).  k_act_l2 writes the level-2
// sums (block b of step^2 elements, zero past the end, which adds nothing), k_act_finish
// chains them per column and adds the result to every target's act_square.  For the usual
// p = 4 the level-2 blocks of the first region are the 256-token blocks of k_xprep, which
// writes them as it passes over the chunk.
__host__ __device__ inline int act_level_power(int64_t count) {
  int cl = 0;
  while (cl < 62 && ((int64_t)1 << cl) < count) ++cl;     // ceil(log2 count); 0 for count <= 1
  return cl / 4 > 4 ? cl / 4 : 4;
}
constexpr int ACT_MAXP = 6;                                 // step <= 64: count < 2^28

template <typename TX>
__device__ __forceinline__ float act_sq_elem(const TX* __restrict__ X, int64_t ldx, int64_t row, int c) {
  const float v = rq_load_elem(X + row * ldx + c);
  return v * v;
}

template <typename TX>
__global__ __launch_bounds__(256) void k_act_l2(const TX* __restrict__ X, int64_t ldx, int c_lo, int V, int lanes,
                                                int64_t count, int lp, float* __restrict__ out, int64_t ldo) {
  __shared__ float l1s[1 << ACT_MAXP][64];
  const int tid = threadIdx.x;
  const int vl = tid & 63, part = tid >> 6;
  const int v = blockIdx.x * 64 + vl;
  const int step = 1 << lp;
  const int64_t base = (int64_t)blockIdx.y << (2 * lp);
  if (v < V) {
    const int c = c_lo + v / lanes, m = v % lanes;
    for (int k = part; k < step; k += 4) {
      const int64_t i0 = base + (int64_t)k * step;
      float s = 0.0f;
      if (i0 + step <= count) {
#pragma unroll 16
        for (int j = 0; j < step; ++j) s = s + act_sq_elem(X, ldx, m + (i0 + j) * lanes, c);
      } else {
        for (int j = 0; j < step; ++j)
          if (i0 + j < count) s = s + act_sq_elem(X, ldx, m + (i0 + j) * lanes, c);
      }
      l1s[k][vl] = s;
    }
  }
  __syncthreads();
  if (part != 0 || v >= V) return;
  float l2 = 0.0f;
  for (int k = 0; k < step; ++k) l2 = l2 + l1s[k][vl];
  out[blockIdx.y * ldo + v] = l2;
}

// Levels 3 and 4 over the level-2 sums of virtual column v (in[b * ldi + v]).
__device__ __forceinline__ float act_chain(const float* __restrict__ in, int64_t ldi, int v, int64_t count, int lp) {
  const int64_t step = (int64_t)1 << lp;
  const int64_t nfull = count >> (2 * lp);
  const bool partial = (count & ((step << lp) - 1)) != 0;
  // The additions stay in sequence order; the loads are issued 16 at a time ahead of them
  // (step = 2^lp is a multiple of 16).
  constexpr int AB = 16;
  float a4 = 0.0f;
  int64_t j = 0;
  for (; j + step <= nfull; j += step) {
    float a3 = 0.0f;
    for (int64_t k0 = 0; k0 < step; k0 += AB) {
      float t[AB];
#pragma unroll
      for (int u = 0; u < AB; ++u) t[u] = in[(j + k0 + u) * ldi + v];
#pragma unroll
      for (int u = 0; u < AB; ++u) a3 = a3 + t[u];
    }
    a4 = a4 + a3;
  }
  float a3 = 0.0f;
  for (; j < nfull; j += AB) {
    float t[AB];
#pragma unroll
    for (int u = 0; u < AB; ++u) t[u] = (j + u < nfull) ? in[(j + u) * ldi + v] : 0.0f;
#pragma unroll
    for (int u = 0; u < AB; ++u)
      if (j + u < nfull) a3 = a3 + t[u];
  }
  const float a12 = partial ? in[nfull * ldi + v] : 0.0f;   // a1 + a2 of the incomplete block
  return (a12 + a3) + a4;
}

template <typename TX>
__device__ __forceinline__ void act_add(const HTargets& tg, int ntarg, int c, float v) {
  for (int g = 0; g < ntarg; ++g)
    if (tg.act[g]) tg.act[g][c] = tg.act[g][c] + v;
}

template <typename TX>
__global__ __launch_bounds__(256) void k_act_finish(const float* __restrict__ in, int64_t ldi, int c_lo, int ncol,
                                                    int lanes, int64_t count, int lp, const TX* __restrict__ X,
                                                    int64_t ldx, int64_t ntok, HTargets tg, int ntarg) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= ncol) return;
  const int c = c_lo + idx;
  float r;
  if (lanes == 1) {
    r = act_chain(in, ldi, idx, count, lp);
  } else {
    float s0 = act_chain(in, ldi, 4 * idx, count, lp);
    for (int64_t t = 4 * count; t < ntok; ++t) s0 = s0 + act_sq_elem(X, ldx, t, c);
    const float s1 = act_chain(in, ldi, 4 * idx + 1, count, lp);
    const float s2 = act_chain(in, ldi, 4 * idx + 2, count, lp);
    const float s3 = act_chain(in, ldi, 4 * idx + 3, count, lp);
    r = ((s0 + s1) + s2) + s3;
  }
  act_add<TX>(tg, ntarg, c, r);
}

// The same reduction without workspace: one thread per column walks its sequence(s) with the
// four running partial sums (slow; used only when the caller gives no workspace).
template <typename TX>
__device__ float act_cascade_seq(const TX* __restrict__ X, int64_t ldx, int c, int m, int lanes, int64_t count) {
  const int lp = act_level_power(count);
  const int64_t step = (int64_t)1 << lp, mask = step - 1;
  float a1 = 0.0f, a2 = 0.0f, a3 = 0.0f, a4 = 0.0f;
  int64_t i = 0;
  while (i + step <= count) {
    for (int64_t j = 0; j < step; ++j, ++i) a1 = a1 + act_sq_elem(X, ldx, m + i * lanes, c);
    a2 = a2 + a1;
    a1 = 0.0f;
    if ((i & (mask << lp)) != 0) continue;
    a3 = a3 + a2;
    a2 = 0.0f;
    if ((i & (mask << (2 * lp))) != 0) continue;
    a4 = a4 + a3;
    a3 = 0.0f;
  }
  for (; i < count; ++i) a1 = a1 + act_sq_elem(X, ldx, m + i * lanes, c);
  return ((a1 + a2) + a3) + a4;
}

template <typename TX>
__global__ __launch_bounds__(256) void k_act_direct(const TX* __restrict__ X, int64_t ntok, int64_t ldx, int C,
                                                    int ca, HTargets tg, int ntarg) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  float r;
  if (c < ca) {
    r = act_cascade_seq(X, ldx, c, 0, 1, ntok);
  } else {
    const int64_t k = ntok / 4;
    float s0 = act_cascade_seq(X, ldx, c, 0, 4, k);
    for (int64_t t = 4 * k; t < ntok; ++t) s0 = s0 + act_sq_elem(X, ldx, t, c);
    const float s1 = act_cascade_seq(X, ldx, c, 1, 4, k);
    const float s2 = act_cascade_seq(X, ldx, c, 2, 4, k);
    const float s3 = act_cascade_seq(X, ldx, c, 3, 4, k);
    r = ((s0 + s1) + s2) + s3;
  }
  act_add<TX>(tg, ntarg, c, r);
}
}  // namespace

namespace {

// finalize_hessian (gptq_plus_utils.py:881-907): divide, symmetrise from the upper triangle,
// sanitise non-finite entries.
// t-th tile of the upper triangle (ti <= tj < nt), row-major, in closed form: row r starts at
// r nt - r (r - 1) / 2.
__device__ __forceinline__ void upper_tile_closed(int t, int nt, int& ti, int& tj) {
  const float b = 2.0f * nt + 1.0f;
  int r = (int)((b - __builtin_sqrtf(b * b - 8.0f * (float)t)) * 0.5f);
  r = max(0, min(r, nt - 1));
  auto start = [nt](int q) { return q * nt - q * (q - 1) / 2; };
  while (r > 0 && start(r) > t) --r;
  while (r + 1 < nt && start(r + 1) <= t) ++r;
  ti = r;
  tj = r + (t - start(r));
}

// The same per element, on 64x64 upper tile pairs: a thread's 16 loads are issued together,
// then the symmetrised values are written to the tile and, through LDS, to its mirror.  (Many
// 32x32 workgroups with 4 elements per thread kept too few loads in flight: ~1.5 TB/s.)
__global__ __launch_bounds__(256) void k_hessian_finalize64(float* __restrict__ H, int C, int nt,
                                                            float h_div, float sal_scale,
                                                            int apply_scale, int sanitize, int* nonfinite) {
  __shared__ float tile[64][65];
  __shared__ int cnt;
  const int g = blockIdx.y;
  int ti, tj;
  upper_tile_closed(blockIdx.x, nt, ti, tj);
  float* Hg = H + (int64_t)g * C * C;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;   // 64 x 4
  if (threadIdx.x == 0) cnt = 0;
  float v[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int i = ti * 64 + ty + 4 * k, j = tj * 64 + tx;
    v[k] = (i < C && j < C) ? Hg[(int64_t)i * C + j] : 0.0f;
  }
  int local = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int y = ty + 4 * k;
    const int i = ti * 64 + y, j = tj * 64 + tx;
    if (i >= C || j >= C) continue;
    if (ti == tj && y > tx) continue;            // lower half of a diagonal tile: mirrored below
    float val = v[k] / h_div;
    if (apply_scale) val = val / sal_scale;
    val = 0.5f * (val + val);                     // 0.5 * (H + H^T) on the symmetric value
    if (!rq_isfinite(val)) {
      if (sanitize) val = 0.0f;
      local += (i == j) ? 1 : 2;
    }
    Hg[(int64_t)i * C + j] = val;
    tile[y][tx] = val;
  }
  __syncthreads();
  // mirror: H[j][i] = H[i][j]; rows of the transposed tile, for coalescing
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const int y = ty + 4 * k;
    const int j = tj * 64 + y, i = ti * 64 + tx;   // element (j, i) takes tile[tx][y]
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

std::atomic<int> g_hmath{RQ_HMATH_SPLIT16X3};   // exact fp32 products by default
// Optional events recorded around the next product-kernel launch (measurement hook).
std::atomic<void*> g_time_start{nullptr}, g_time_stop{nullptr};

// Record the hook's start event before the product kernel; returns the stop event to record
// after it (nullptr when no hook is set).  Each pair is used once.
hipEvent_t timing_begin(hipStream_t s) {
  void* a = g_time_start.exchange(nullptr);
  void* b = g_time_stop.exchange(nullptr);
  if (!a || !b) return nullptr;
  if (hipEventRecord(reinterpret_cast<hipEvent_t>(a), s) != hipSuccess) return nullptr;
  return reinterpret_cast<hipEvent_t>(b);
}

// Concurrent workgroups of a Hessian kernel on the current device (CUs x occupancy).
template <typename K>
int kernel_slots(K kfn, int threads, int which) {
  static int cache[3][64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[which][dev] > 0) return cache[which][dev];
  int cus = 0, occ = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kfn, threads, 0) != hipSuccess) return 0;
  cache[which][dev] = cus * occ;
  return cache[which][dev];
}
int hessian_slots() { return kernel_slots(k_hessian_accum<__half>, HTHREADS, 0); }
int hessian_slots32() { return kernel_slots(k_hessian_accum<float>, HTHREADS, 2); }
int accum_slots(int x_dtype) { return x_dtype == RQ_F32 ? hessian_slots32() : hessian_slots(); }
int split_slots() { return kernel_slots(k_hessian_split<__half, 3>, XTHREADS, 1); }

// Items of the last, partly filled round and their slice count: the most slices that still
// fit the tail into one round (S = slots / tail, S <= maxS, at least 4 token slabs per slice).
// Measured at C = 4096 (tails of 32, 64, 96 and 136 items on 256 slots: best S = 6-8, 3-4, 2 and
// 1-3) and 14336 (240 items: 1).  Splitting further, into more rounds, loses: besides each
// slice's partial tile and the last slice's reduction, the power-limited clock rises when fewer
// CUs are busy, so a tail on part of the GPU costs less than its idle share.  The split kernels
// reduce up to 16 slices, the fp32 kernel up to 8.
void tail_split(int64_t total, int64_t nslab, int slots, int maxS, int* tail, int* S) {
  *tail = 0;
  *S = 1;
  if (slots <= 0 || total <= 0) return;
  const int64_t t = total % slots;
  if (t == 0) return;
  int64_t s = slots / t;
  if (s > maxS) s = maxS;
  while (s > 1 && nslab < 4 * s) --s;
  if (s > 1) {
    *tail = (int)t;
    *S = (int)s;
  }
}

int64_t align256(int64_t b) { return ((b + 255) / 256) * 256; }

// Workspace layout: one int counter per possible tail item at a fixed place (the start, sized
// for the larger slot count of the two kernels), so launches with different tails and either
// kernel can share one workspace; then the act_square level-2 sums; then the partial tiles;
// then (split kernel) the X pass.
int64_t hessian_cnt_bytes() {
  const int a = hessian_slots(), b = split_slots();
  return align256((int64_t)(a > b ? a : b) * 4);
}

// act_square regions of a call: the one-sequence columns [0, ca) and the interleaved columns
// [ca, C) (four sequences each).
struct ActPlan {
  int ca;
  int lp_main, lp_tail;
  int64_t nl2_main, nl2_tail, off_tail, bytes;
};

ActPlan act_plan(int64_t ntok, int C) {
  ActPlan P;
  P.ca = (C / 32) * 32;
  P.lp_main = act_level_power(ntok);
  P.lp_tail = act_level_power(ntok / 4);
  P.nl2_main = (ntok + ((int64_t)1 << (2 * P.lp_main)) - 1) >> (2 * P.lp_main);
  P.nl2_tail = (ntok / 4 + ((int64_t)1 << (2 * P.lp_tail)) - 1) >> (2 * P.lp_tail);
  P.off_tail = align256(P.nl2_main * P.ca * 4);
  P.bytes = P.off_tail + align256(P.nl2_tail * 4 * (int64_t)(C - P.ca) * 4);
  return P;
}

int64_t act_off() { return hessian_cnt_bytes(); }

// fp32-MFMA kernel: counters, act_square sums, then the tail slices' partial tiles.
int64_t hessian_ws_bytes(int64_t ntok, int C, int64_t tail, int S) {
  return act_off() + act_plan(ntok, C).bytes + (tail > 0 ? tail * S * (int64_t)HPART * 4 : 0);
}

// act_square of one call into every target's act pointer (no-op when none has one).
// l2_main: the first region's level-2 sums already written by k_xprep (row stride C; only
// valid for lp_main == 4), else nullptr.  ws_act: the act region of the workspace, or nullptr
// (then the slow one-pass kernel runs).
template <typename TX>
int launch_act_square_t(const TX* x, int64_t ntok, int64_t ldx, int C, const HTargets& tg, int ntarg,
                        const float* l2_main, char* ws_act, hipStream_t s) {
  bool any = false;
  for (int g = 0; g < ntarg; ++g) any = any || tg.act[g];
  if (!any || ntok <= 0) return RQ_OK;
  const ActPlan P = act_plan(ntok, C);
  if (P.lp_main > ACT_MAXP) return RQ_EINVAL;
  if (!ws_act) {
    hipLaunchKernelGGL(k_act_direct<TX>, dim3((C + 255) / 256), dim3(256), 0, s, x, ntok, ldx, C, P.ca, tg, ntarg);
    RQ_CHECK_LAUNCH();
    return RQ_OK;
  }
  if (P.ca > 0) {
    const float* l2 = l2_main;
    int64_t ld = C;
    if (!l2 || P.lp_main != 4) {
      float* out = reinterpret_cast<float*>(ws_act);
      hipLaunchKernelGGL(k_act_l2<TX>, dim3((P.ca + 63) / 64, (unsigned)P.nl2_main), dim3(256), 0, s, x, ldx, 0,
                         P.ca, 1, ntok, P.lp_main, out, (int64_t)P.ca);
      RQ_CHECK_LAUNCH();
      l2 = out;
      ld = P.ca;
    }
    hipLaunchKernelGGL(k_act_finish<TX>, dim3((P.ca + 255) / 256), dim3(256), 0, s, l2, ld, 0, P.ca, 1, ntok,
                       P.lp_main, x, ldx, ntok, tg, ntarg);
    RQ_CHECK_LAUNCH();
  }
  if (P.ca < C) {
    const int nc = C - P.ca, V = 4 * nc;
    float* out = reinterpret_cast<float*>(ws_act + P.off_tail);
    if (P.nl2_tail > 0) {
      hipLaunchKernelGGL(k_act_l2<TX>, dim3((V + 63) / 64, (unsigned)P.nl2_tail), dim3(256), 0, s, x, ldx, P.ca,
                         V, 4, ntok / 4, P.lp_tail, out, (int64_t)V);
      RQ_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(k_act_finish<TX>, dim3((nc + 255) / 256), dim3(256), 0, s, out, (int64_t)V, P.ca, nc, 4,
                       ntok / 4, P.lp_tail, x, ldx, ntok, tg, ntarg);
    RQ_CHECK_LAUNCH();
  }
  return RQ_OK;
}

int launch_act_square(const void* x, int x_dtype, int64_t ntok, int64_t ldx, int C, const HTargets& tg, int ntarg,
                      const float* l2_main, char* ws_act, hipStream_t s) {
  if (x_dtype == RQ_F16)
    return launch_act_square_t(static_cast<const __half*>(x), ntok, ldx, C, tg, ntarg, l2_main, ws_act, s);
  if (x_dtype == RQ_BF16)
    return launch_act_square_t(static_cast<const __hip_bfloat16*>(x), ntok, ldx, C, tg, ntarg, l2_main, ws_act, s);
  return launch_act_square_t(static_cast<const float*>(x), ntok, ldx, C, tg, ntarg, l2_main, ws_act, s);
}

struct SplitLayout {
  int64_t ntok_p, nchunk, off_part, off_xt, off_st, off_m, off_a, off_s, off_scale, bytes;
};

SplitLayout split_layout(int64_t ntok, int C, int ntarg, int64_t tail, int S) {
  SplitLayout L;
  L.ntok_p = ((ntok + XTOK - 1) / XTOK) * XTOK;
  L.nchunk = L.ntok_p / XTOK;
  L.off_part = act_off() + act_plan(ntok, C).bytes;
  L.off_xt = L.off_part + align256(tail * S * (int64_t)XPART * 4);
  L.off_st = L.off_xt + align256((int64_t)((C + 31) / 32) * 32 * L.ntok_p * 2);
  L.off_m = L.off_st + align256((int64_t)ntarg * L.ntok_p * 4);
  L.off_a = L.off_m + align256(L.nchunk * C * 4);
  L.off_s = L.off_a + align256(L.nchunk * C * 4);
  L.off_scale = L.off_s + align256(L.nchunk * HMAXT * 4);
  L.bytes = L.off_scale + align256((int64_t)ntarg * C * 4);
  return L;
}

void split_items(int C, int ntarg, int* nt, int* ntiles, int64_t* total) {
  *nt = (C + XT - 1) / XT;
  *ntiles = *nt * (*nt + 1) / 2;
  *total = (int64_t)*ntiles * ntarg;
}

// Workspace bytes the split kernel needs for one launch of `ntarg` targets.
int64_t split_ws_need(int64_t ntok, int C, int ntarg) {
  int nt, ntiles;
  int64_t total;
  split_items(C, ntarg, &nt, &ntiles, &total);
  int tail = 0, S = 1;
  const int64_t ntok_p = ((ntok + XTOK - 1) / XTOK) * XTOK;
  tail_split(total, ntok_p / 16, split_slots(), 16, &tail, &S);
  return split_layout(ntok, C, ntarg, tail, S).bytes;
}

// Whole items per launch of the split kernel, in rounds of `slots` workgroups (see launch_split).
// One round per launch: all its workgroups start together and do equal work, so the targets of
// a tile and the tiles of a super-row read their X strips through the XCD's L2 in step.  In one
// launch of many rounds the workgroups' start times drift apart from round to round (25 rounds
// per configs[2] down_proj call), and they re-read the strips from HBM.  Measured on the
// configs[2] layer (two boxes, two A/B passes each): HBM fetch of the split kernel -40 % per
// layer; layer time -2.0 / -1.8 / -1.5 / -1.6 % with 1 / 2 / 3 / 4 rounds per launch, -1.0 /
// -0.2 % with 3 / 5 rounds on the other box.
constexpr int XSEG_ROUNDS = 1;

int launch_split(const void* x, int x_dtype, int64_t ntok, int64_t ldx, int C, const HTargets& tg,
                 int ntarg, void* ws, int64_t ws_bytes, hipStream_t s) {
  int nt, ntiles;
  int64_t total;
  split_items(C, ntarg, &nt, &ntiles, &total);
  if (total > 0x7fffffff / 8) return RQ_EINVAL;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && (((size_t)ldx * 2) % 16 == 0);
  int tail = 0, S = 1;
  SplitLayout L = split_layout(ntok, C, ntarg, 0, 1);
  const int64_t nks = L.ntok_p / 16;
  tail_split(total, nks, split_slots(), 16, &tail, &S);
  L = split_layout(ntok, C, ntarg, tail, S);
  if (ws_bytes < L.bytes) {                       // no room for the slices: whole items only
    tail = 0;
    S = 1;
    L = split_layout(ntok, C, ntarg, 0, 1);
  }
  char* wb = reinterpret_cast<char*>(ws);
  uint16_t* xt = reinterpret_cast<uint16_t*>(wb + L.off_xt);
  float* sT = reinterpret_cast<float*>(wb + L.off_st);
  float* mpart = reinterpret_cast<float*>(wb + L.off_m);
  float* apart = reinterpret_cast<float*>(wb + L.off_a);
  float* spart = reinterpret_cast<float*>(wb + L.off_s);
  float* scale = reinterpret_cast<float*>(wb + L.off_scale);
  dim3 pgrid((C + XPC - 1) / XPC, (unsigned)L.nchunk), fgrid((C + XF_COLS - 1) / XF_COLS);
  if (x_dtype == RQ_F16)
    hipLaunchKernelGGL(k_xprep<__half>, pgrid, dim3(256), 0, s, (const __half*)x, ntok, ldx, C, vec_ok, xt,
                       nks, tg, ntarg, sT, L.ntok_p, mpart, apart, spart);
  else
    hipLaunchKernelGGL(k_xprep<__hip_bfloat16>, pgrid, dim3(256), 0, s, (const __hip_bfloat16*)x, ntok, ldx,
                       C, vec_ok, xt, nks, tg, ntarg, sT, L.ntok_p, mpart, apart, spart);
  RQ_CHECK_LAUNCH();
  hipLaunchKernelGGL(k_xfinish, fgrid, dim3(256), 0, s, C, (int)L.nchunk, ntarg, mpart, spart, scale, nullptr);
  RQ_CHECK_LAUNCH();
  {
    const int rc = launch_act_square(x, x_dtype, ntok, ldx, C, tg, ntarg, apart, wb + act_off(), s);
    if (rc) return rc;
  }
  const int full = (int)(total - tail);
  int* cnt = tail > 0 ? reinterpret_cast<int*>(ws) : nullptr;
  float* wsf = tail > 0 ? reinterpret_cast<float*>(wb + L.off_part) : nullptr;
  const int od_items = nt * (nt - 1) / 2 * ntarg;
  // Segments of XSEG_ROUNDS rounds of whole items, each a launch of its own (the tail's slices
  // ride with the last): the kernel boundary brings every XCD's workgroups back in step.
  const int slots = split_slots();
  const int rounds = slots > 0 ? full / slots : 0;
  const int nseg = (XSEG_ROUNDS > 0 && rounds > XSEG_ROUNDS) ? (rounds + XSEG_ROUNDS - 1) / XSEG_ROUNDS : 1;
  hipEvent_t stop = timing_begin(s);
  const dim3 block(XTHREADS);
  for (int q = 0; q < nseg; ++q) {
    const int p0 = (nseg == 1) ? 0 : (int)((int64_t)rounds * q / nseg) * slots;
    const int p1 = (q + 1 == nseg) ? full : (int)((int64_t)rounds * (q + 1) / nseg) * slots;
    const int segn = p1 - p0;
    const int od_seg = std::min(segn, std::max(0, od_items - p0));
    const dim3 grid((unsigned)(segn + (q + 1 == nseg ? (int64_t)tail * S : 0)));
    if (x_dtype == RQ_F16 && g_hmath.load() == RQ_HMATH_SPLIT16X3)
      hipLaunchKernelGGL((k_hessian_split<__half, 3>), grid, block, 0, s, xt, C, sT, L.ntok_p, scale, tg, ntarg,
                         nt, ntiles, nks, p0, segn, od_seg, full, S, wsf, cnt);
    else if (x_dtype == RQ_F16)
      hipLaunchKernelGGL((k_hessian_split<__half, 2>), grid, block, 0, s, xt, C, sT, L.ntok_p, scale, tg, ntarg,
                         nt, ntiles, nks, p0, segn, od_seg, full, S, wsf, cnt);
    else
      hipLaunchKernelGGL((k_hessian_split<__hip_bfloat16, 3>), grid, block, 0, s, xt, C, sT, L.ntok_p, scale, tg,
                         ntarg, nt, ntiles, nks, p0, segn, od_seg, full, S, wsf, cnt);
    RQ_CHECK_LAUNCH();
  }
  if (stop && hipEventRecord(stop, s) != hipSuccess) return RQ_EHIP;
  return RQ_OK;
}

// fp32 X workspace: the split layout plus the hi / lo row pieces, the fp32 column fragments and
// the per-column row scales.
struct SplitLayout32 {
  SplitLayout base;
  int64_t off_xh, off_xl, off_xc, off_rs, bytes;
};

SplitLayout32 split_layout32(int64_t ntok, int C, int ntarg, int64_t tail, int S) {
  SplitLayout32 L;
  L.base = split_layout(ntok, C, ntarg, tail, S);
  const int64_t frag16 = align256((int64_t)((C + 31) / 32) * 32 * L.base.ntok_p * 2);
  L.off_xh = L.base.bytes;
  L.off_xl = L.off_xh + frag16;
  L.off_xc = L.off_xl + frag16;
  L.off_rs = L.off_xc + 2 * frag16;
  L.bytes = L.off_rs + align256((int64_t)C * 4);
  return L;
}

int split32_slots() { return kernel_slots(k_hessian_split32, XTHREADS, 1); }

int64_t split32_ws_need(int64_t ntok, int C, int ntarg) {
  int nt, ntiles;
  int64_t total;
  split_items(C, ntarg, &nt, &ntiles, &total);
  int tail = 0, S = 1;
  const int64_t ntok_p = ((ntok + XTOK - 1) / XTOK) * XTOK;
  tail_split(total, ntok_p / 16, split32_slots(), 16, &tail, &S);
  return split_layout32(ntok, C, ntarg, tail, S).bytes;
}

int launch_split32(const float* x, int64_t ntok, int64_t ldx, int C, const HTargets& tg, int ntarg, void* ws,
                   int64_t ws_bytes, hipStream_t s) {
  int nt, ntiles;
  int64_t total;
  split_items(C, ntarg, &nt, &ntiles, &total);
  if (total > 0x7fffffff / 8) return RQ_EINVAL;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && (((size_t)ldx * 4) % 16 == 0);
  int tail = 0, S = 1;
  SplitLayout32 L = split_layout32(ntok, C, ntarg, 0, 1);
  const int64_t nks = L.base.ntok_p / 16;
  tail_split(total, nks, split32_slots(), 16, &tail, &S);
  L = split_layout32(ntok, C, ntarg, tail, S);
  if (ws_bytes < L.bytes) {                       // no room for the slices: whole items only
    tail = 0;
    S = 1;
    L = split_layout32(ntok, C, ntarg, 0, 1);
  }
  char* wb = reinterpret_cast<char*>(ws);
  uint16_t* xh = reinterpret_cast<uint16_t*>(wb + L.off_xh);
  uint16_t* xl = reinterpret_cast<uint16_t*>(wb + L.off_xl);
  float* xc = reinterpret_cast<float*>(wb + L.off_xc);
  float* rs = reinterpret_cast<float*>(wb + L.off_rs);
  float* sT = reinterpret_cast<float*>(wb + L.base.off_st);
  float* mpart = reinterpret_cast<float*>(wb + L.base.off_m);
  float* apart = reinterpret_cast<float*>(wb + L.base.off_a);
  float* spart = reinterpret_cast<float*>(wb + L.base.off_s);
  float* scale = reinterpret_cast<float*>(wb + L.base.off_scale);
  dim3 pgrid((C + XPC - 1) / XPC, (unsigned)L.base.nchunk), fgrid((C + XF_COLS - 1) / XF_COLS);
  hipLaunchKernelGGL(k_xprep32, pgrid, dim3(256), 0, s, x, ntok, ldx, C, vec_ok, reinterpret_cast<float4*>(xc),
                     nks, tg, ntarg, sT, L.base.ntok_p, mpart, apart, spart);
  RQ_CHECK_LAUNCH();
  hipLaunchKernelGGL(k_xfinish, fgrid, dim3(256), 0, s, C, (int)L.base.nchunk, ntarg, mpart, spart, scale, rs);
  RQ_CHECK_LAUNCH();
  const int64_t nfrag = (int64_t)((C + 31) / 32) * nks;
  hipLaunchKernelGGL(k_xrows32, dim3((unsigned)((nfrag * 64 + 255) / 256)), dim3(256), 0, s,
                     reinterpret_cast<const float4*>(xc), nfrag, C, nks, rs, reinterpret_cast<uint4*>(xh),
                     reinterpret_cast<uint4*>(xl));
  RQ_CHECK_LAUNCH();
  {
    const int rc = launch_act_square(x, RQ_F32, ntok, ldx, C, tg, ntarg, apart, wb + act_off(), s);
    if (rc) return rc;
  }
  const int full = (int)(total - tail);
  int* cnt = tail > 0 ? reinterpret_cast<int*>(ws) : nullptr;
  float* wsf = tail > 0 ? reinterpret_cast<float*>(wb + L.base.off_part) : nullptr;
  dim3 grid((unsigned)(full + (int64_t)tail * S)), block(XTHREADS);
  hipEvent_t stop = timing_begin(s);
  hipLaunchKernelGGL(k_hessian_split32, grid, block, 0, s, xh, xl, xc, C, sT, L.base.ntok_p, scale, rs, tg, ntarg,
                     nt, ntiles, nks, full, S, wsf, cnt);
  RQ_CHECK_LAUNCH();
  if (stop && hipEventRecord(stop, s) != hipSuccess) return RQ_EHIP;
  return RQ_OK;
}

int launch_hessian(const void* x, int x_dtype, int64_t ntok, int64_t ldx, int C, const HTargets& tg,
                   int ntarg, void* ws, int64_t ws_bytes, hipStream_t s) {
  const bool aligned = ws && ((reinterpret_cast<uintptr_t>(ws) & 255) == 0);
  if (x_dtype != RQ_F32 && g_hmath.load() != RQ_HMATH_FP32 && aligned &&
      ws_bytes >= split_layout(ntok, C, ntarg, 0, 1).bytes)
    return launch_split(x, x_dtype, ntok, ldx, C, tg, ntarg, ws, ws_bytes, s);
  // fp32 X: the split kernel (products within ~2^-20.5) only in the opt-in two-piece mode; by
  // default the fp32 MFMA kernel below forms the reference's products exactly
  if (x_dtype == RQ_F32 && g_hmath.load() == RQ_HMATH_SPLIT16 && aligned &&
      ws_bytes >= split_layout32(ntok, C, ntarg, 0, 1).bytes)
    return launch_split32(static_cast<const float*>(x), ntok, ldx, C, tg, ntarg, ws, ws_bytes, s);
  const int nt = (C + HT - 1) / HT;
  const int ntiles = nt * (nt + 1) / 2;
  const int64_t total = (int64_t)ntiles * ntarg;
  if (total > 0x7fffffff / 8) return RQ_EINVAL;
  const size_t esz = (x_dtype == RQ_F32) ? 4 : 2;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && (((size_t)ldx * esz) % 16 == 0);
  const bool have_act_ws = aligned && ws_bytes >= hessian_ws_bytes(ntok, C, 0, 1);
  {
    const int rc = launch_act_square(x, x_dtype, ntok, ldx, C, tg, ntarg, nullptr,
                                     have_act_ws ? reinterpret_cast<char*>(ws) + act_off() : nullptr, s);
    if (rc) return rc;
  }
  int tail = 0, S = 1;
  if (aligned) tail_split(total, (ntok + HKC - 1) / HKC, accum_slots(x_dtype), 8, &tail, &S);
  if (tail > 0 && ws_bytes < hessian_ws_bytes(ntok, C, tail, S)) {
    tail = 0;                                     // no room: whole items only
    S = 1;
  }
  const int full = (int)(total - tail);
  int* cnt = tail > 0 ? reinterpret_cast<int*>(ws) : nullptr;
  float* wsf = tail > 0 ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + act_off() + act_plan(ntok, C).bytes)
                        : nullptr;
  dim3 grid((unsigned)(full + (int64_t)tail * S)), block(HTHREADS);
  hipEvent_t stop = timing_begin(s);
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
  if (stop && hipEventRecord(stop, s) != hipSuccess) return RQ_EHIP;
  return RQ_OK;
}

}  // namespace

extern "C" int rq_hessian_timing_events(void* start_event, void* stop_event) {
  if ((start_event == nullptr) != (stop_event == nullptr)) return RQ_EINVAL;
  g_time_stop.store(stop_event);
  g_time_start.store(start_event);
  return RQ_OK;
}

extern "C" int rq_hessian_math(int mode) {
  if (mode < 0) return g_hmath.load();
  if (mode != RQ_HMATH_SPLIT16 && mode != RQ_HMATH_FP32 && mode != RQ_HMATH_SPLIT16X3) return RQ_EINVAL;
  return g_hmath.exchange(mode);
}

extern "C" int64_t rq_hessian_workspace_bytes(int64_t ntok, int C, int ntargets, int x_dtype) {
  if (ntok < 0 || C <= 0 || ntargets <= 0) return RQ_EINVAL;
  if (x_dtype != RQ_F16 && x_dtype != RQ_BF16 && x_dtype != RQ_F32) return RQ_EINVAL;
  const int nt = (C + HT - 1) / HT;
  int64_t need = 0;
  for (int t0 = 0; t0 < ntargets; t0 += HMAXT) {   // per launch of at most 32 targets
    const int n = (ntargets - t0 < HMAXT) ? (ntargets - t0) : HMAXT;
    int tail = 0, S = 1;
    tail_split((int64_t)nt * (nt + 1) / 2 * n, (ntok + HKC - 1) / HKC, accum_slots(x_dtype), 8, &tail, &S);
    int64_t b = hessian_ws_bytes(ntok, C, tail, S);
    const int64_t bs = x_dtype == RQ_F32 ? split32_ws_need(ntok, C, n) : split_ws_need(ntok, C, n);
    if (bs > b) b = bs;
    if (b > need) need = b;
  }
  return need;
}

// Scratch of the no-allocation variant: one array per device (the code object's own copy on
// each GPU), held until the process ends.  Host code never passes the array's name to a
// kernel: it takes the device address from hipGetSymbolAddress once per device.
static __device__ __align__(256) uint8_t scratch[RQ_NOALLOC_SCRATCH_BYTES];

namespace {

__global__ void k_zero_words(uint32_t* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

constexpr int SCRATCH_MAXDEV = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[SCRATCH_MAXDEV] = {};

// Device address of the current device's scratch.  The first call on a device looks it up and
// clears the tail-slice counters (the kernels return them to zero after every launch) with a
// fill kernel on the caller's stream, ahead of the launches that use them.
int scratch_of_current_device(hipStream_t s, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return RQ_EHIP;
  if (dev < 0 || dev >= SCRATCH_MAXDEV) return RQ_EINVAL;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return RQ_EHIP;
    const int64_t words = hessian_cnt_bytes() / 4;
    hipLaunchKernelGGL(k_zero_words, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s,
                       static_cast<uint32_t*>(p), words);
    RQ_CHECK_LAUNCH();
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return RQ_OK;
}

}  // namespace

extern "C" int rq_hessian_accum_noalloc(const void* x, int x_dtype, int64_t ntok, int64_t ldx, int C,
                                        const float* sal, int64_t ld_sal, int G, float* H, float* act_sq,
                                        void* stream) {
  if (!x || !sal || !H || C <= 0 || G <= 0 || ntok < 0 || ldx < C || ld_sal < G) return RQ_EINVAL;
  if (x_dtype != RQ_F16 && x_dtype != RQ_BF16 && x_dtype != RQ_F32) return RQ_EINVAL;
  if (ntok == 0) return RQ_OK;
  // the least scratch the kernel rq_hessian_accum would choose needs (whole items only)
  const int n = G < HMAXT ? G : HMAXT;
  const int64_t need = (x_dtype != RQ_F32 && g_hmath.load() != RQ_HMATH_FP32)
                           ? split_layout(ntok, C, n, 0, 1).bytes
                           : hessian_ws_bytes(ntok, C, 0, 1);
  if (need > (int64_t)RQ_NOALLOC_SCRATCH_BYTES) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  void* ws = nullptr;
  const int rc = scratch_of_current_device(s, &ws);
  if (rc) return rc;
  return rq_hessian_accum(x, x_dtype, ntok, ldx, C, sal, ld_sal, G, H, act_sq, ws,
                          (int64_t)RQ_NOALLOC_SCRATCH_BYTES, stream);
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
                                   double sal_scale, double seq_len, int sanitize, int* nonfinite,
                                   void* stream) {
  if (!H || C <= 0 || G <= 0 || !(h_div > 0) || !(seq_len > 0)) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int nt = (C + 63) / 64;
  const int ntiles = nt * (nt + 1) / 2;
  // torch divides a float tensor by a Python scalar in float: a / (float)b (CPU kernel).
  hipLaunchKernelGGL(k_hessian_finalize64, dim3(ntiles, G), dim3(256), 0, s, H, C, nt, (float)h_div,
                     (float)sal_scale, sal_scale != 1.0 ? 1 : 0, sanitize ? 1 : 0, nonfinite);
  RQ_CHECK_LAUNCH();
  if (act_sq) {
    hipLaunchKernelGGL(k_scale_vec, dim3((C + 255) / 256), dim3(256), 0, s, act_sq, C, (float)seq_len);
    RQ_CHECK_LAUNCH();
  }
  return RQ_OK;
}
