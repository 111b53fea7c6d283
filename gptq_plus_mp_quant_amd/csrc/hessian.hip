// Saliency-weighted multi-group Hessian accumulation (GPTQPlus.add_batch,
// gptq_utils/gptq_plus_utils.py:798-857) and its finalisation (finalize_hessian, :859-908).
//
// H[g] += X^T diag(s_g) X is computed as a symmetric rank-k update: only 128x128 tiles on or
// above the diagonal are formed (the mirrored half is never computed), one workgroup per
// (tile, group).  Each workgroup streams 32-token slabs of X[:, I] and X[:, J] (fp16/bf16/fp32)
// through double-buffered LDS, converting to fp32 once; the per-token saliency s[t, g] is
// folded into the B operand as it is written to LDS (the reference's `weighted` tensor,
// fl32(x * s), is never materialised).  Products run on v_mfma_f32_32x32x2f32 with fp32
// accumulation; each 64x64 quarter of the tile belongs to one wave (2x2 MFMA blocks).
// The diagonal tiles of group 0 also accumulate act_square = sum_t x^2.  No atomics: every
// output element has exactly one owner, so results are bitwise reproducible run to run.
#include "rq_common.h"

namespace {

constexpr int HT = 128;      // output tile edge
constexpr int HKC = 32;      // tokens per LDS slab
constexpr int HTHREADS = 256;

struct XLoad {
  float v[2][16];            // [side][16 consecutive columns]
};

template <typename TX>
__device__ __forceinline__ void load_slab(const TX* __restrict__ X, int64_t ntok, int64_t ldx,
                                          int C, int64_t t0, int I0, int J0, bool diag,
                                          bool vec_ok, XLoad& r) {
  const int tid = threadIdx.x;
  const int k = tid >> 3;             // token within slab (0..31)
  const int c0 = (tid & 7) * 16;      // first of 16 columns
  const int64_t t = t0 + k;
#pragma unroll
  for (int side = 0; side < 2; ++side) {
    if (side == 1 && diag) break;
    const int col = (side == 0 ? I0 : J0) + c0;
    if (t < ntok && vec_ok && col + 16 <= C) {
      const TX* p = X + t * ldx + col;
      if constexpr (sizeof(TX) == 2) {
        const uint4* q = reinterpret_cast<const uint4*>(p);
        uint4 u0 = q[0], u1 = q[1];
        const TX* h0 = reinterpret_cast<const TX*>(&u0);
        const TX* h1 = reinterpret_cast<const TX*>(&u1);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          r.v[side][e] = rq_load_elem(h0 + e);
          r.v[side][8 + e] = rq_load_elem(h1 + e);
        }
      } else {
        const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float4 f = q[e];
          r.v[side][4 * e + 0] = f.x;
          r.v[side][4 * e + 1] = f.y;
          r.v[side][4 * e + 2] = f.z;
          r.v[side][4 * e + 3] = f.w;
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int cc = col + e;
        r.v[side][e] = (t < ntok && cc < C) ? rq_load_elem(X + t * ldx + cc) : 0.0f;
      }
    }
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

template <typename TX>
__global__ __launch_bounds__(HTHREADS, 2) void k_hessian_accum(
    const TX* __restrict__ X, int64_t ntok, int64_t ldx, int C, const float* __restrict__ sal,
    int64_t ld_sal, int G, float* __restrict__ H, float* __restrict__ act_sq, int nt, int ntiles,
    bool vec_ok) {
  __shared__ float As[2][HKC][HT];
  __shared__ float Bs[2][HKC][HT];

  // XCD-aware order: consecutive hardware workgroup ids land on different XCDs (round
  // robin over 8); give each XCD a contiguous run of logical ids so neighbouring tiles,
  // which share X column strips, share that XCD's L2.
  const int total = ntiles * G;
  const int b = blockIdx.x;
  const int per = total / 8, rem8 = total % 8;
  const int xcd = b % 8, idx = b / 8;
  const int logical = (xcd < rem8) ? xcd * (per + 1) + idx : rem8 * (per + 1) + (xcd - rem8) * per + idx;
  const int g = logical % G;
  int ti, tj;
  upper_tile(logical / G, nt, ti, tj);
  const int I0 = ti * HT, J0 = tj * HT;
  const bool diag = (ti == tj);
  const bool want_act = diag && (g == 0) && (act_sq != nullptr);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int lk = tid >> 3;            // token row this thread stages
  const int lc = (tid & 7) * 16;      // first column this thread stages

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  float actp[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) actp[e] = 0.0f;

  const int64_t nslab = (ntok + HKC - 1) / HKC;
  XLoad r;

  auto stage = [&](int buf, int64_t t0) {
    const int64_t t = t0 + lk;
    const float s = (t < ntok) ? sal[t * ld_sal + g] : 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const float xa = r.v[0][e];
      As[buf][lk][lc + e] = xa;
      const float xb = diag ? xa : r.v[1][e];
      Bs[buf][lk][lc + e] = xb * s;       // fl32(x * s): the reference's `weighted`
      if (want_act) actp[e] += xa * xa;
    }
  };

  load_slab<TX>(X, ntok, ldx, C, 0, I0, J0, diag, vec_ok, r);
  stage(0, 0);
  __syncthreads();

  for (int64_t sidx = 0; sidx < nslab; ++sidx) {
    const int buf = (int)(sidx & 1);
    const bool more = (sidx + 1) < nslab;
    if (more) load_slab<TX>(X, ntok, ldx, C, (sidx + 1) * HKC, I0, J0, diag, vec_ok, r);
#pragma unroll
    for (int ks = 0; ks < HKC / 2; ++ks) {
      const int k = 2 * ks + (lane >> 5);
      const float a0 = As[buf][k][wr * 64 + (lane & 31)];
      const float a1 = As[buf][k][wr * 64 + 32 + (lane & 31)];
      const float b0 = Bs[buf][k][wc * 64 + (lane & 31)];
      const float b1 = Bs[buf][k][wc * 64 + 32 + (lane & 31)];
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
    }
    if (more) stage(buf ^ 1, (sidx + 1) * HKC);
    __syncthreads();
  }

  // H[g][I0 + i][J0 + j] += acc   (32x32 block layout: i = 8*(e/4) + 4*(lane/32) + e%4, j = lane%32)
  float* Hg = H + (int64_t)g * C * C;
#pragma unroll
  for (int bi = 0; bi < 2; ++bi)
#pragma unroll
    for (int bj = 0; bj < 2; ++bj)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = I0 + wr * 64 + bi * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int j = J0 + wc * 64 + bj * 32 + (lane & 31);
        if (i < C && j < C) {
          float* p = Hg + (int64_t)i * C + j;
          *p = *p + acc[bi][bj][e];
        }
      }

  if (want_act) {
    // Sum the 32 per-token-row partials of each column in a fixed order (As is free now).
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 16; ++e) As[0][lk][lc + e] = actp[e];
    __syncthreads();
    if (tid < HT && I0 + tid < C) {
      float s = 0.0f;
      for (int q = 0; q < HKC; ++q) s += As[0][q][tid];
      act_sq[I0 + tid] += s;
    }
  }
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

extern "C" int rq_hessian_accum(const void* x, int x_dtype, int64_t ntok, int64_t ldx, int C,
                                const float* sal, int64_t ld_sal, int G, float* H, float* act_sq,
                                void* stream) {
  if (!x || !sal || !H || C <= 0 || G <= 0 || ntok < 0 || ldx < C || ld_sal < G) return RQ_EINVAL;
  if (x_dtype != RQ_F16 && x_dtype != RQ_BF16 && x_dtype != RQ_F32) return RQ_EINVAL;
  if (ntok == 0) return RQ_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int nt = (C + HT - 1) / HT;
  const int ntiles = nt * (nt + 1) / 2;
  const int64_t total = (int64_t)ntiles * G;
  if (total > 0x7fffffff) return RQ_EINVAL;
  const size_t esz = (x_dtype == RQ_F32) ? 4 : 2;
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && (((size_t)ldx * esz) % 16 == 0);
  dim3 grid((unsigned)total), block(HTHREADS);
  if (x_dtype == RQ_F16)
    hipLaunchKernelGGL(k_hessian_accum<__half>, grid, block, 0, s, (const __half*)x, ntok, ldx, C,
                       sal, ld_sal, G, H, act_sq, nt, ntiles, vec_ok);
  else if (x_dtype == RQ_BF16)
    hipLaunchKernelGGL(k_hessian_accum<__hip_bfloat16>, grid, block, 0, s,
                       (const __hip_bfloat16*)x, ntok, ldx, C, sal, ld_sal, G, H, act_sq, nt,
                       ntiles, vec_ok);
  else
    hipLaunchKernelGGL(k_hessian_accum<float>, grid, block, 0, s, (const float*)x, ntok, ldx, C,
                       sal, ld_sal, G, H, act_sq, nt, ntiles, vec_ok);
  RQ_CHECK_LAUNCH();
  return RQ_OK;
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
