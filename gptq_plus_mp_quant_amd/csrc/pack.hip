// Packed export of the quantized weight: integer codes as an nbits-wide bitstream per row
// plus a [ngroups, R] scale table and a per-column group index.
//
// The reference keeps its export as two full fp32 [R, C] tensors (int_weight and scale,
// gptq_utils/gptq_plus_utils.py:1866-1871); this format carries the same information in
// nbits/32 + a fraction of the space.  Codes are what fasterquant produced
// (clamp(rint(w/s), -(maxq+1), maxq)); they are stored offset by 2^(nbits-1), so nbits is
// `bits` for sym and `bits + 1` for asym (the asym fake_quantize clamps to the signed range
// [-(maxq+1), maxq], quant_utils.py:477, which needs one more bit).
//
// Row r is a little-endian bitstream: code c occupies bits [c*nbits, (c+1)*nbits) of the
// row, bit b of the row is bit (b & 31) of 32-bit word (b >> 5).  Words past the last code
// are zero-padded.  Dequantisation: Q[r, c] = scales[g_idx[c]][r] * (field(r, c) - 2^(nbits-1)).
//
// k_pack_rows: one thread per output word reads the <= 32/nbits + 1 codes overlapping it
// (through invperm when the codes are still in act_order's permuted order), so the codes
// are read once and every word is written once: 2·R·C + R·C·nbits/8 bytes, HBM-bound.
// k_unpack_dequant: one thread per weight, reading the one or two words its field spans.
#include "rq_common.h"

namespace {

__global__ __launch_bounds__(256) void k_pack_rows(const int16_t* __restrict__ codes, int R, int C,
                                                   int64_t ldc, const int64_t* __restrict__ invperm,
                                                   int nbits, uint32_t* __restrict__ out,
                                                   int64_t ldo, int words, int* __restrict__ range_flag) {
  const int w = blockIdx.x * 256 + threadIdx.x;
  if (w >= words) return;
  const int half = 1 << (nbits - 1);
  const uint32_t mask = (1u << nbits) - 1u;
  const int64_t bit0 = (int64_t)w * 32;
  const int c0 = (int)(bit0 / nbits);
  const int c1 = min(C - 1, (int)((bit0 + 31) / nbits));
  int bad = 0;
  for (int r = blockIdx.y; r < R; r += gridDim.y) {
    const int16_t* crow = codes + (int64_t)r * ldc;
    uint32_t word = 0;
    for (int c = c0; c <= c1; ++c) {
      const int64_t j = invperm ? invperm[c] : c;
      const int v = (int)crow[j] + half;
      bad |= (v < 0) | (v > (int)mask);
      const uint32_t u = (uint32_t)v & mask;
      const int shift = (int)((int64_t)c * nbits - bit0);   // in (-nbits, 32)
      word |= shift >= 0 ? (u << shift) : (u >> (-shift));
    }
    out[(int64_t)r * ldo + w] = word;
  }
  if (bad && range_flag) atomicOr(range_flag, 1);
}

template <typename TQ>
__global__ __launch_bounds__(256) void k_unpack_dequant(const uint32_t* __restrict__ packed, int R,
                                                        int C, int64_t ldp, int nbits,
                                                        const float* __restrict__ scales,
                                                        int64_t lds, const int32_t* __restrict__ g_idx,
                                                        TQ* __restrict__ q_out, int64_t ldq,
                                                        int16_t* __restrict__ codes_out) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  const int half = 1 << (nbits - 1);
  const uint32_t mask = (1u << nbits) - 1u;
  const int64_t bit = (int64_t)c * nbits;
  const int64_t wi = bit >> 5;
  const int off = (int)(bit & 31);
  const bool spans = off + nbits > 32;
  const int64_t grp = g_idx ? g_idx[c] : 0;
  for (int r = blockIdx.y; r < R; r += gridDim.y) {
    const uint32_t* prow = packed + (int64_t)r * ldp;
    uint32_t v = prow[wi] >> off;
    if (spans) v |= prow[wi + 1] << (32 - off);
    const int code = (int)(v & mask) - half;
    if (codes_out) codes_out[(int64_t)r * C + c] = (int16_t)code;
    if (q_out) {
      float qf = scales[grp * lds + r] * (float)code;
      // keep fl32(s * code) and the cast to the output type as two roundings (the
      // compiler would otherwise fuse them into one v_fma_mix), as in the write-back
      asm volatile("" : "+v"(qf));
      q_out[(int64_t)r * ldq + c] = rq_cast<TQ>(qf);
    }
  }
}

inline int rows_grid(int rows) { return rows < 1024 ? rows : 1024; }

}  // namespace

extern "C" int64_t rq_packed_words_per_row(int C, int nbits) {
  if (C <= 0 || nbits < 2 || nbits > 16) return RQ_EINVAL;
  return ((int64_t)C * nbits + 31) / 32;
}

extern "C" int rq_pack_codes(const int16_t* codes, int R, int C, int64_t ldc, const int64_t* invperm,
                             int nbits, uint32_t* out, int64_t ldo, int* range_flag, void* stream) {
  if (!codes || !out || R <= 0 || C <= 0 || ldc < C || nbits < 2 || nbits > 16) return RQ_EINVAL;
  const int64_t words = rq_packed_words_per_row(C, nbits);
  if (ldo < words || words > INT32_MAX) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((unsigned)((words + 255) / 256), rows_grid(R)), block(256);
  hipLaunchKernelGGL(k_pack_rows, grid, block, 0, s, codes, R, C, ldc, invperm, nbits, out, ldo,
                     (int)words, range_flag);
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}

extern "C" int rq_unpack_dequant(const uint32_t* packed, int R, int C, int64_t ldp, int nbits,
                                 const float* scales, int64_t lds, const int32_t* g_idx, void* q_out,
                                 int q_dtype, int64_t ldq, int16_t* codes_out, void* stream) {
  if (!packed || R <= 0 || C <= 0 || nbits < 2 || nbits > 16) return RQ_EINVAL;
  if (ldp < rq_packed_words_per_row(C, nbits)) return RQ_EINVAL;
  if (!q_out && !codes_out) return RQ_EINVAL;
  if (q_out && (!scales || lds < R || ldq < C)) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((C + 255) / 256, rows_grid(R)), block(256);
  if (!q_out || q_dtype == RQ_F16)
    hipLaunchKernelGGL(k_unpack_dequant<__half>, grid, block, 0, s, packed, R, C, ldp, nbits, scales,
                       lds, g_idx, (__half*)q_out, ldq, codes_out);
  else if (q_dtype == RQ_BF16)
    hipLaunchKernelGGL(k_unpack_dequant<__hip_bfloat16>, grid, block, 0, s, packed, R, C, ldp, nbits,
                       scales, lds, g_idx, (__hip_bfloat16*)q_out, ldq, codes_out);
  else if (q_dtype == RQ_F32)
    hipLaunchKernelGGL(k_unpack_dequant<float>, grid, block, 0, s, packed, R, C, ldp, nbits, scales,
                       lds, g_idx, (float*)q_out, ldq, codes_out);
  else
    return RQ_EINVAL;
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}
