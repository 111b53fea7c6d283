// Quantizer parameters, per-subgroup gathers and the final write-back.
//  - rq_find_params:      WeightQuantizer.find_params, per-channel min/max (utils/quant_utils.py:390-421),
//                         also per static column group (gptq_utils/gptq_plus_utils.py:994-1002) and
//                         find_params_weight_groupwise (utils/quant_utils.py:333-388, clip_zero = 0)
//  - rq_prepare_subgroup: row slice, dead columns, act_order gathers of W, G and H (:1033-1050)
//  - rq_writeback:        un-permute, dequantize, cast to the layer dtype, export buffers (:1850-1896)
// All of these are HBM-bound gathers / reductions.
#include <type_traits>

#include "rq_common.h"

namespace {

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = rq_nan_min(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = rq_nan_max(v, __shfl_xor(v, o, 64));
  return v;
}

// One wavefront per (row, group).
template <typename TW>
__global__ __launch_bounds__(256) void k_find_params(const TW* __restrict__ w, int R, int C,
                                                     int64_t ldw, int gs, float maxq, int sym, int clip_zero,
                                                     float* __restrict__ scale,
                                                     float* __restrict__ zero) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int grp = blockIdx.y;
  if (r >= R) return;
  const int c0 = grp * gs;
  const int c1 = min(C, c0 + gs);
  const TW* row = w + (int64_t)r * ldw;
  float mn = __builtin_inff(), mx = -__builtin_inff();
  // lane order c = c0 + lane, + 64, ... (the order decides which zero a min / max of +0 and -0
  // keeps); 8 loads in flight per lane
  int c = c0 + lane;
  for (; c + 7 * 64 < c1; c += 8 * 64) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = rq_load_elem(row + c + 64 * u);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      mn = rq_nan_min(mn, v[u]);
      mx = rq_nan_max(mx, v[u]);
    }
  }
  for (; c < c1; c += 64) {
    const float v = rq_load_elem(row + c);
    mn = rq_nan_min(mn, v);
    mx = rq_nan_max(mx, v);
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  if (lane == 0) {
    float s, z;
    rq_params_from_minmax(mn, mx, maxq, sym, &s, &z, clip_zero);
    scale[(int64_t)grp * R + r] = s;
    zero[(int64_t)grp * R + r] = z;
  }
}

// WeightQuantizer.find_params with mse=True (utils/quant_utils.py:408-448): min/max start,
// then a maxshrink*grid x maxshrink*grid shrink grid over (xmin, xmax); each candidate's row
// error sum |q - x|^norm is reduced in a fixed order and the first strict minimum wins
// (clip_zero = 0: the groupwise search of :354-386, from the group's own min / max).
// One 256-thread workgroup per (row, group).
template <typename TW>
__global__ __launch_bounds__(256) void k_find_params_mse(const TW* __restrict__ w, int R, int C,
                                                         int64_t ldw, int gs, float maxq, int sym,
                                                         int clip_zero, float norm, int grid, int steps,
                                                         float* __restrict__ scale,
                                                         float* __restrict__ zero) {
  __shared__ float red[256];
  __shared__ float red2[256];
  const int tid = threadIdx.x;
  const int r = blockIdx.x, grp = blockIdx.y;
  const int c0 = grp * gs;
  const int c1 = min(C, c0 + gs);
  const TW* row = w + (int64_t)r * ldw;
  float mn = __builtin_inff(), mx = -__builtin_inff();
  for (int c = c0 + tid; c < c1; c += 256) {
    const float v = rq_load_elem(row + c);
    mn = rq_nan_min(mn, v);
    mx = rq_nan_max(mx, v);
  }
  red[tid] = mn;
  red2[tid] = mx;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) {
      red[tid] = rq_nan_min(red[tid], red[tid + o]);
      red2[tid] = rq_nan_max(red2[tid], red2[tid + o]);
    }
    __syncthreads();
  }
  float xmin = clip_zero ? rq_nan_min(red[0], 0.0f) : red[0];
  float xmax = clip_zero ? rq_nan_max(red2[0], 0.0f) : red2[0];
  if (!sym && xmin == 0.0f && xmax == 0.0f) {
    xmin = -1.0f;
    xmax = 1.0f;
  }
  float bscale, bzero;
  rq_params_from_minmax(red[0], red2[0], maxq, sym, &bscale, &bzero, clip_zero);
  float best = __builtin_inff();
  for (int i = 0; i < steps; ++i) {
    const float fi = (float)(1.0 - (double)i / (double)grid);
    for (int j = 0; j < steps; ++j) {
      const float fj = (float)(1.0 - (double)j / (double)grid);
      const float xmin1 = fi * xmin, xmax1 = fj * xmax;
      float s1, z1;
      if (sym) {
        s1 = rq_clamp_min(rq_nan_max(fabsf(xmin1), xmax1), 1e-5f) / maxq;
        z1 = 0.0f;
      } else {
        s1 = (xmax1 - xmin1) / maxq;
        z1 = __builtin_rintf(-xmin1 / s1);
      }
      float part = 0.0f;
      for (int c = c0 + tid; c < c1; c += 256) {
        const float x = rq_load_elem(row + c);
        float q;
        if (sym) {
          q = s1 * rq_quant_code(x, s1, -(maxq + 1.0f), maxq);
        } else {
          float t = __builtin_rintf(x / s1) + z1;
          t = (t < 0.0f) ? 0.0f : t;
          t = (t > maxq) ? maxq : t;
          q = s1 * (t - z1);
        }
        part += powf(fabsf(q - x), norm);
      }
      __syncthreads();                  // red[] of the previous candidate fully read
      red[tid] = part;
      __syncthreads();
      for (int o = 128; o > 0; o >>= 1) {
        if (tid < o) red[tid] = red[tid] + red[tid + o];
        __syncthreads();
      }
      const float err = red[0];
      if (err < best) {                 // same value in every thread: uniform update
        best = err;
        bscale = s1;
        bzero = z1;
      }
    }
  }
  if (tid == 0) {
    scale[(int64_t)grp * R + r] = bscale;
    zero[(int64_t)grp * R + r] = bzero;
  }
}

template <typename TW>
__global__ __launch_bounds__(256) void k_gather_w(const TW* __restrict__ w, int64_t ldw,
                                                  const float* __restrict__ Hg, int R_s, int C,
                                                  const int64_t* __restrict__ perm,
                                                  float* __restrict__ out, int64_t ldo) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= C) return;
  const int64_t p = perm ? perm[j] : j;
  const bool dead = Hg[p * C + p] == 0.0f;
  for (int r = blockIdx.y; r < R_s; r += gridDim.y)
    out[(int64_t)r * ldo + j] = dead ? 0.0f : rq_load_elem(w + (int64_t)r * ldw + p);
}

__global__ __launch_bounds__(256) void k_gather_g(const float* __restrict__ g, int64_t ldg, int R_s,
                                                  int C, const int64_t* __restrict__ perm,
                                                  float* __restrict__ out, int64_t ldo) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= C) return;
  const int64_t p = perm ? perm[j] : j;
  for (int r = blockIdx.y; r < R_s; r += gridDim.y) out[(int64_t)r * ldo + j] = g[(int64_t)r * ldg + p];
}

// Row-staged gathers.  A workgroup copies `nr` whole source rows into LDS (16-byte loads when
// the rows allow, 8 in flight per thread), then writes the output rows in order, column j
// taking LDS element perm[j]: every source byte is read from HBM once and the writes are
// coalesced.  The column kernels above (the fallback for rows too wide for LDS) read one
// element per thread from anywhere in its row, fetching each row's cache lines once per
// 256-column workgroup.  Row stride in LDS: C elements rounded up to 16 bytes.
template <typename TS>
__host__ __device__ constexpr int padded_cols(int C) {
  return (int)(((int64_t)C * (int64_t)sizeof(TS) + 15) / 16 * 16 / (int64_t)sizeof(TS));
}

template <int NT, typename TS>
__device__ __forceinline__ void stage_rows(const TS* __restrict__ src, int64_t lds, int r0, int nr, int C,
                                           bool vec, uint8_t* smem) {
  const int tid = threadIdx.x;
  const int cpad = padded_cols<TS>(C);
  if (vec) {
    const int n16 = (int)((int64_t)C * sizeof(TS) / 16);
    const int rb = cpad * (int)sizeof(TS);
    const int tot = nr * n16;
    for (int q0 = tid; q0 < tot; q0 += NT * 8) {
      uint4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int q = q0 + NT * u;
        if (q < tot)
          v[u] = reinterpret_cast<const uint4*>(src + (int64_t)(r0 + q / n16) * lds)[q % n16];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int q = q0 + NT * u;
        if (q < tot) reinterpret_cast<uint4*>(smem + (int64_t)(q / n16) * rb)[q % n16] = v[u];
      }
    }
  } else {
    TS* buf = reinterpret_cast<TS*>(smem);
    for (int rr = 0; rr < nr; ++rr)
      for (int q = tid; q < C; q += NT) buf[(int64_t)rr * cpad + q] = src[(int64_t)(r0 + rr) * lds + q];
  }
}

// Source column of each output column for the row-staged gathers: idx_w[j] = perm[j], or -1
// for a dead column (H_g[perm[j], perm[j]] == 0: W's column is zeroed), idx_g[j] = perm[j].
// Written once per subgroup into H_sub's first 2 C words, which k_gather_h_rows overwrites
// afterwards on the same stream; the row gathers then read one coalesced index per column
// instead of perm[j] and a diagonal element of H_g each.
__global__ __launch_bounds__(256) void k_gather_index(const float* __restrict__ Hg, int C,
                                                      const int64_t* __restrict__ perm, int32_t* __restrict__ idx_w,
                                                      int32_t* __restrict__ idx_g) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= C) return;
  const int64_t p = perm ? perm[j] : j;
  idx_w[j] = (Hg[p * C + p] == 0.0f) ? -1 : (int32_t)p;
  idx_g[j] = (int32_t)p;
}

// out[r, j] = src[r, idx[j]] (0 where idx[j] < 0) for rows r0 .. r0 + nr - 1: k_gather_w /
// k_gather_g by rows.  NT threads (1024 for rows that leave room for only one or two
// workgroups per CU); GU columns' index loads in flight per thread.
constexpr int GU = 8;
template <int NT, typename TS>
__global__ __launch_bounds__(NT) void k_gather_rows(const TS* __restrict__ src, int64_t lds, int rows, int C,
                                                    int rpw, bool vec, const int32_t* __restrict__ idx,
                                                    float* __restrict__ out, int64_t ldo) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int r0 = blockIdx.x * rpw;
  const int nr = min(rpw, rows - r0);
  stage_rows<NT>(src, lds, r0, nr, C, vec, smem);
  __syncthreads();
  const TS* buf = reinterpret_cast<const TS*>(smem);
  const int cpad = padded_cols<TS>(C);
  for (int j0 = threadIdx.x; j0 < C; j0 += NT * GU) {
    int p[GU];
#pragma unroll
    for (int u = 0; u < GU; ++u) {
      const int j = j0 + NT * u;
      p[u] = (j < C) ? idx[j] : 0;
    }
    for (int rr = 0; rr < nr; ++rr)
#pragma unroll
      for (int u = 0; u < GU; ++u) {
        const int j = j0 + NT * u;
        if (j < C)
          out[(int64_t)(r0 + rr) * ldo + j] = (p[u] < 0) ? 0.0f : rq_load_elem(buf + (int64_t)rr * cpad + p[u]);
      }
  }
}

__global__ __launch_bounds__(256) void k_gather_h(const float* __restrict__ Hg, int C,
                                                  const int64_t* __restrict__ perm,
                                                  float* __restrict__ out) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= C) return;
  const int64_t pj = perm ? perm[j] : j;
  for (int i = blockIdx.y; i < C; i += gridDim.y) {
    const int64_t pi = perm ? perm[i] : i;
    float v = Hg[pi * C + pj];
    if (i == j && v == 0.0f) v = 1.0f;            // H_sub[dead, dead] = 1
    out[(int64_t)i * C + j] = v;
  }
}

// P H P by rows: workgroup i stages source row perm[i] in LDS with 16-byte loads (the whole
// row, C floats), then writes output row i coalesced, column j taking LDS word perm[j].
// Each source row is read from HBM once; the column-gather kernel above re-read every source
// row's cache lines once per 256-column workgroup.  Dynamic LDS: C * 4 bytes (112 KB at
// C = 28672, one workgroup per CU), so there both loops keep GR_U loads per thread in flight;
// small rows run unrolled once with 256 threads and several workgroups per CU instead.
template <int GR_THREADS, int GR_U>
__global__ __launch_bounds__(GR_THREADS) void k_gather_h_rows(const float* __restrict__ Hg, int C,
                                                              const int64_t* __restrict__ perm,
                                                              float* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) float row[];
  const int i = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t pi = perm ? perm[i] : i;
  const float* src = Hg + pi * C;
  if ((C & 3) == 0) {
    const float4* s4 = reinterpret_cast<const float4*>(src);
    const int n4 = C / 4;
    for (int q0 = tid; q0 < n4; q0 += GR_THREADS * GR_U) {
      float4 v[GR_U];
#pragma unroll
      for (int u = 0; u < GR_U; ++u) {
        const int q = q0 + u * GR_THREADS;
        if (q < n4) v[u] = s4[q];
      }
#pragma unroll
      for (int u = 0; u < GR_U; ++u) {
        const int q = q0 + u * GR_THREADS;
        if (q < n4) reinterpret_cast<float4*>(row)[q] = v[u];
      }
    }
  } else {
    for (int q = tid; q < C; q += GR_THREADS) row[q] = src[q];
  }
  __syncthreads();
  float* dst = out + (int64_t)i * C;
  for (int j0 = tid; j0 < C; j0 += GR_THREADS * GR_U) {
    int pj[GR_U];
#pragma unroll
    for (int u = 0; u < GR_U; ++u) {
      const int j = j0 + u * GR_THREADS;
      pj[u] = (j < C) ? (perm ? (int)perm[j] : j) : 0;
    }
#pragma unroll
    for (int u = 0; u < GR_U; ++u) {
      const int j = j0 + u * GR_THREADS;
      if (j < C) {
        float v = row[pj[u]];
        if (j == i && v == 0.0f) v = 1.0f;        // H_sub[dead, dead] = 1
        dst[j] = v;
      }
    }
  }
}

template <typename TQ>
__global__ __launch_bounds__(256) void k_writeback(const int16_t* __restrict__ codes, int R, int C,
                                                   const int64_t* __restrict__ invperm, int qmode,
                                                   const float* __restrict__ scale,
                                                   const int32_t* __restrict__ col_group,
                                                   const float* __restrict__ dyn_scale, int bs,
                                                   TQ* __restrict__ q_out, int64_t ldq,
                                                   float* __restrict__ w_int_out,
                                                   float* __restrict__ scale_out,
                                                   int* __restrict__ nan_flag) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  const int64_t j = invperm ? invperm[c] : c;
  int nan_seen = 0;
  for (int r = blockIdx.y; r < R; r += gridDim.y) {
    const int16_t ci = codes[(int64_t)r * C + j];
    const float code = (ci == RQ_CODE_NAN) ? __builtin_nanf("") : (float)ci;   // NaN weight
    float s;
    if (qmode == RQ_QMODE_CHANNEL) s = scale[r];
    else if (qmode == RQ_QMODE_STATIC) s = scale[(int64_t)col_group[j] * R + r];
    else s = dyn_scale[(j / bs) * (int64_t)R + r];
    float qf = s * code;
    // Keep fl32(s * code) as its own rounding step: without the barrier the compiler folds
    // the multiply and the fp16 conversion into v_fma_mixlo_f16 (a single rounding), which
    // differs from torch's (scale * q).to(float16) on exact fp16 midpoints.
    asm volatile("" : "+v"(qf));
    const TQ q = rq_cast<TQ>(qf);
    q_out[(int64_t)r * ldq + c] = q;
    const float qback = (float)q;
    nan_seen |= (qback != qback);
    if (w_int_out) w_int_out[(int64_t)r * C + c] = code;
    if (scale_out) scale_out[(int64_t)r * C + c] = s;
  }
  if (nan_seen && nan_flag) atomicOr(nan_flag, 1);
}

// k_writeback by rows: the workgroup's rows of codes staged in LDS (as k_gather_rows), then
// each output row written in order, column c taking LDS element invperm[c]; the same
// arithmetic as k_writeback.
template <int NT, typename TQ>
__global__ __launch_bounds__(NT) void k_writeback_rows(const int16_t* __restrict__ codes, int R, int C, int rpw,
                                                        bool vec, const int64_t* __restrict__ invperm, int qmode,
                                                        const float* __restrict__ scale,
                                                        const int32_t* __restrict__ col_group,
                                                        const float* __restrict__ dyn_scale, int bs,
                                                        TQ* __restrict__ q_out, int64_t ldq,
                                                        float* __restrict__ w_int_out,
                                                        float* __restrict__ scale_out,
                                                        int* __restrict__ nan_flag) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int r0 = blockIdx.x * rpw;
  const int nr = min(rpw, R - r0);
  stage_rows<NT>(codes, C, r0, nr, C, vec, smem);
  __syncthreads();
  const int16_t* buf = reinterpret_cast<const int16_t*>(smem);
  const int cpad = padded_cols<int16_t>(C);
  int nan_seen = 0;
  constexpr int WU = 4;   // columns whose index loads are in flight per thread
  for (int c0 = threadIdx.x; c0 < C; c0 += NT * WU) {
    int64_t jj[WU], gb[WU];
#pragma unroll
    for (int u = 0; u < WU; ++u) {
      const int c = c0 + NT * u;
      jj[u] = (c < C) ? (invperm ? invperm[c] : c) : 0;
    }
#pragma unroll
    for (int u = 0; u < WU; ++u)
      gb[u] = (qmode == RQ_QMODE_STATIC)  ? (int64_t)col_group[jj[u]] * R
              : (qmode == RQ_QMODE_DYNAMIC) ? (jj[u] / bs) * (int64_t)R
                                            : 0;
    for (int rr = 0; rr < nr; ++rr) {
#pragma unroll
      for (int u = 0; u < WU; ++u) {
        const int c = c0 + NT * u;
        if (c >= C) continue;
        const int64_t j = jj[u], gbase = gb[u];
        const int r = r0 + rr;
        const int16_t ci = buf[(int64_t)rr * cpad + j];
        const float code = (ci == RQ_CODE_NAN) ? __builtin_nanf("") : (float)ci;   // NaN weight
        float s;
        if (qmode == RQ_QMODE_CHANNEL) s = scale[r];
        else if (qmode == RQ_QMODE_STATIC) s = scale[gbase + r];
        else s = dyn_scale[gbase + r];
        float qf = s * code;
        asm volatile("" : "+v"(qf));   // fl32(s * code), then the cast: two roundings (k_writeback)
        const TQ q = rq_cast<TQ>(qf);
        q_out[(int64_t)r * ldq + c] = q;
        const float qback = (float)q;
        nan_seen |= (qback != qback);
        if (w_int_out) w_int_out[(int64_t)r * C + c] = code;
        if (scale_out) scale_out[(int64_t)r * C + c] = s;
      }
    }
  }
  if (nan_seen && nan_flag) atomicOr(nan_flag, 1);
}

inline int rows_grid(int rows) { return rows < 1024 ? rows : 1024; }

// Rows per workgroup and LDS bytes of a row-staged launch over `rows` rows of C elements of
// `esize` bytes: enough workgroups to keep ~1024 in the grid, at most 4 rows and 64 KB; 0 when
// one row does not fit the LDS a workgroup may have (then the column kernels run).
template <typename K>
inline size_t rows_launch(K kernel, int rows, int C, int esize, int* rpw) {
  const size_t rb = (size_t)(((int64_t)C * esize + 15) / 16 * 16);
  int n = rows / 1024;
  n = n < 1 ? 1 : (n > 4 ? 4 : n);
  while (n > 1 && (size_t)n * rb > 64 * 1024) --n;
  const size_t bytes = (size_t)n * rb;
  if (bytes > 64 * 1024 &&
      (bytes > 160 * 1024 ||
       hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) != hipSuccess))
    return 0;
  *rpw = n;
  return bytes;
}

// 16-byte row loads: the row length and stride are whole 16-byte units and the base is aligned.
inline bool rows_vec(const void* p, int64_t ld, int C, int esize) {
  return ((int64_t)C * esize) % 16 == 0 && (ld * esize) % 16 == 0 && ((uintptr_t)p & 15) == 0;
}

// 256 threads per workgroup while a row is at most 32 KB, else 1024 (LDS then holds one or
// two workgroups per CU).
inline bool rows_wide(int C, int esize) { return (int64_t)C * esize > 32 * 1024; }

template <typename TS>
inline bool launch_gather_rows(const TS* src, int64_t lds, int rows, int C, const int32_t* idx, float* out,
                               int64_t ldo, hipStream_t s) {
  int rpw = 1;
  const bool vec = rows_vec(src, lds, C, (int)sizeof(TS));
  if (rows_wide(C, (int)sizeof(TS))) {
    const size_t bytes = rows_launch(k_gather_rows<1024, TS>, rows, C, (int)sizeof(TS), &rpw);
    if (!bytes) return false;
    hipLaunchKernelGGL((k_gather_rows<1024, TS>), dim3((rows + rpw - 1) / rpw), dim3(1024), bytes, s, src, lds,
                       rows, C, rpw, vec, idx, out, ldo);
  } else {
    const size_t bytes = rows_launch(k_gather_rows<256, TS>, rows, C, (int)sizeof(TS), &rpw);
    if (!bytes) return false;
    hipLaunchKernelGGL((k_gather_rows<256, TS>), dim3((rows + rpw - 1) / rpw), dim3(256), bytes, s, src, lds,
                       rows, C, rpw, vec, idx, out, ldo);
  }
  return true;
}

}  // namespace

extern "C" int rq_find_params(const void* w, int w_dtype, int R, int C, int64_t ldw, int group_size,
                              int maxq, int sym, int clip_zero, float* scale, float* zero, void* stream) {
  if (!w || !scale || !zero || R <= 0 || C <= 0 || ldw < C || maxq <= 0) return RQ_EINVAL;
  const int gs = group_size > 0 ? group_size : C;
  const int ng = (C + gs - 1) / gs;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((R + 3) / 4, ng), block(256);
  if (w_dtype == RQ_F16)
    hipLaunchKernelGGL(k_find_params<__half>, grid, block, 0, s, (const __half*)w, R, C, ldw, gs,
                       (float)maxq, sym, clip_zero, scale, zero);
  else if (w_dtype == RQ_BF16)
    hipLaunchKernelGGL(k_find_params<__hip_bfloat16>, grid, block, 0, s, (const __hip_bfloat16*)w, R,
                       C, ldw, gs, (float)maxq, sym, clip_zero, scale, zero);
  else if (w_dtype == RQ_F32)
    hipLaunchKernelGGL(k_find_params<float>, grid, block, 0, s, (const float*)w, R, C, ldw, gs,
                       (float)maxq, sym, clip_zero, scale, zero);
  else
    return RQ_EINVAL;
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}

extern "C" int rq_find_params_mse(const void* w, int w_dtype, int R, int C, int64_t ldw,
                                  int group_size, int maxq, int sym, int clip_zero, double norm, int grid,
                                  double maxshrink, float* scale, float* zero, void* stream) {
  if (!w || !scale || !zero || R <= 0 || C <= 0 || ldw < C || maxq <= 0 || grid <= 0) return RQ_EINVAL;
  const int gs = group_size > 0 ? group_size : C;
  const int ng = (C + gs - 1) / gs;
  const int steps = (int)(maxshrink * grid);   // int(self.maxshrink * self.grid)
  if (steps <= 0) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 g(R, ng), block(256);
  if (w_dtype == RQ_F16)
    hipLaunchKernelGGL(k_find_params_mse<__half>, g, block, 0, s, (const __half*)w, R, C, ldw, gs,
                       (float)maxq, sym, clip_zero, (float)norm, grid, steps, scale, zero);
  else if (w_dtype == RQ_BF16)
    hipLaunchKernelGGL(k_find_params_mse<__hip_bfloat16>, g, block, 0, s, (const __hip_bfloat16*)w, R,
                       C, ldw, gs, (float)maxq, sym, clip_zero, (float)norm, grid, steps, scale, zero);
  else if (w_dtype == RQ_F32)
    hipLaunchKernelGGL(k_find_params_mse<float>, g, block, 0, s, (const float*)w, R, C, ldw, gs,
                       (float)maxq, sym, clip_zero, (float)norm, grid, steps, scale, zero);
  else
    return RQ_EINVAL;
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}

extern "C" int rq_prepare_subgroup(const void* w, int w_dtype, int64_t ldw, const float* grad,
                                   int64_t ldg, const float* H_g, int R_s, int C,
                                   const int64_t* perm, float* W_sub, int64_t ld_wsub, float* G_sub,
                                   int64_t ld_gsub, float* H_sub, void* stream) {
  if (!w || !H_g || !W_sub || !H_sub || R_s <= 0 || C <= 0 || ldw < C || ld_wsub < C) return RQ_EINVAL;
  if (grad && (!G_sub || ldg < C || ld_gsub < C)) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 gw((C + 255) / 256, rows_grid(R_s)), block(256);
  // the source-column indices of the row gathers, in H_sub's first 2 C words (C >= 2), which
  // the H gather below overwrites after the W / G gathers have read them (same stream)
  int32_t* idx_w = reinterpret_cast<int32_t*>(H_sub);
  int32_t* idx_g = idx_w + C;
  const bool by_rows = C >= 2 && (uintptr_t)H_sub % 4 == 0;
  if (by_rows) {
    hipLaunchKernelGGL(k_gather_index, dim3((C + 255) / 256), block, 0, s, H_g, C, perm, idx_w, idx_g);
    RQ_CHECK_LAUNCH();
  }
  if (w_dtype == RQ_F16) {
    if (!by_rows || !launch_gather_rows((const __half*)w, ldw, R_s, C, idx_w, W_sub, ld_wsub, s))
      hipLaunchKernelGGL(k_gather_w<__half>, gw, block, 0, s, (const __half*)w, ldw, H_g, R_s, C, perm,
                         W_sub, ld_wsub);
  } else if (w_dtype == RQ_BF16) {
    if (!by_rows || !launch_gather_rows((const __hip_bfloat16*)w, ldw, R_s, C, idx_w, W_sub, ld_wsub, s))
      hipLaunchKernelGGL(k_gather_w<__hip_bfloat16>, gw, block, 0, s, (const __hip_bfloat16*)w, ldw, H_g,
                         R_s, C, perm, W_sub, ld_wsub);
  } else if (w_dtype == RQ_F32) {
    if (!by_rows || !launch_gather_rows((const float*)w, ldw, R_s, C, idx_w, W_sub, ld_wsub, s))
      hipLaunchKernelGGL(k_gather_w<float>, gw, block, 0, s, (const float*)w, ldw, H_g, R_s, C, perm,
                         W_sub, ld_wsub);
  } else {
    return RQ_EINVAL;
  }
  RQ_CHECK_LAUNCH();
  if (grad) {
    if (!by_rows || !launch_gather_rows(grad, ldg, R_s, C, idx_g, G_sub, ld_gsub, s))
      hipLaunchKernelGGL(k_gather_g, gw, block, 0, s, grad, ldg, R_s, C, perm, G_sub, ld_gsub);
    RQ_CHECK_LAUNCH();
  }
  const size_t row_bytes = (size_t)C * sizeof(float);
  if (row_bytes <= 64 * 1024 ||
      (row_bytes <= 160 * 1024 &&
       hipFuncSetAttribute((const void*)k_gather_h_rows<512, 8>, hipFuncAttributeMaxDynamicSharedMemorySize,
                           (int)row_bytes) == hipSuccess)) {
    if (C >= 8192)
      hipLaunchKernelGGL((k_gather_h_rows<512, 8>), dim3(C), dim3(512), row_bytes, s, H_g, C, perm, H_sub);
    else
      hipLaunchKernelGGL((k_gather_h_rows<256, 1>), dim3(C), dim3(256), row_bytes, s, H_g, C, perm, H_sub);
  } else {
    hipLaunchKernelGGL(k_gather_h, dim3((C + 255) / 256, rows_grid(C)), block, 0, s, H_g, C, perm, H_sub);
  }
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}

extern "C" int rq_writeback(const int16_t* codes, int R, int C, const int64_t* invperm, int qmode,
                            const float* scale, const int32_t* col_group, const float* dyn_scale,
                            int blocksize, void* q_out, int q_dtype, int64_t ldq, float* w_int_out,
                            float* scale_out, int* nan_flag, void* stream) {
  if (!codes || !q_out || R <= 0 || C <= 0 || ldq < C) return RQ_EINVAL;
  if (qmode == RQ_QMODE_CHANNEL && !scale) return RQ_EINVAL;
  if (qmode == RQ_QMODE_STATIC && (!scale || !col_group)) return RQ_EINVAL;
  if (qmode == RQ_QMODE_DYNAMIC && (!dyn_scale || blocksize <= 0)) return RQ_EINVAL;
  if (qmode < 0 || qmode > 2) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((C + 255) / 256, rows_grid(R)), block(256);
  // by rows when a row of codes fits the LDS of a workgroup, else the column kernel
  auto run = [&](auto* q) -> int {
    typedef typename std::remove_pointer<decltype(q)>::type TQ;
    int rpw = 1;
    const bool vec = rows_vec(codes, C, C, (int)sizeof(int16_t));
    const bool wide = rows_wide(C, (int)sizeof(int16_t));
    const size_t bytes = wide ? rows_launch(k_writeback_rows<1024, TQ>, R, C, (int)sizeof(int16_t), &rpw)
                              : rows_launch(k_writeback_rows<256, TQ>, R, C, (int)sizeof(int16_t), &rpw);
    if (bytes && wide)
      hipLaunchKernelGGL((k_writeback_rows<1024, TQ>), dim3((R + rpw - 1) / rpw), dim3(1024), bytes, s, codes, R,
                         C, rpw, vec, invperm, qmode, scale, col_group, dyn_scale, blocksize, q, ldq, w_int_out,
                         scale_out, nan_flag);
    else if (bytes)
      hipLaunchKernelGGL((k_writeback_rows<256, TQ>), dim3((R + rpw - 1) / rpw), block, bytes, s, codes, R, C,
                         rpw, vec, invperm, qmode, scale, col_group, dyn_scale, blocksize, q, ldq, w_int_out,
                         scale_out, nan_flag);
    else
      hipLaunchKernelGGL(k_writeback<TQ>, grid, block, 0, s, codes, R, C, invperm, qmode, scale, col_group,
                         dyn_scale, blocksize, q, ldq, w_int_out, scale_out, nan_flag);
    return RQ_OK;
  };
  if (q_dtype == RQ_F16)
    run((__half*)q_out);
  else if (q_dtype == RQ_BF16)
    run((__hip_bfloat16*)q_out);
  else if (q_dtype == RQ_F32)
    run((float*)q_out);
  else
    return RQ_EINVAL;
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}
