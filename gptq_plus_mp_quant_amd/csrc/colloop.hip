// The fasterquant block loop (gptq_utils/gptq_plus_utils.py:1169-1372) and the trailing
// (outer) update (:1500-1570), all subgroups in one launch each, for the frozen and the two
// surrogate g_update modes.
//
// k_quant_block: rows are independent, so each row of the block is owned by 16 lanes (one DPP
// row); lane t holds columns t, t+16, ..., t+112 of the row in 8 registers (W1, GHinv1, Z1),
// 16 rows per 256-thread workgroup, one subgroup per workgroup, so 4096 rows keep every SIMD
// busy.  The B x B block of Hinv (upper) sits in LDS as Hp[i][t][k] = Hinv1[i][16k + t], so a
// lane reads its 8 entries of row i with two 16-byte loads.  Column i = 16m + r is quantised by
// lane r of every row, its error is broadcast to the row with one DPP row_newbcast move, and
// every lane applies the rank-1 update to its own columns.  The 128-column loop is fully
// unrolled, so every register index is a compile-time constant.  Arithmetic follows the
// reference op by op (no contraction, IEEE divide, round-half-even):
//   code = clamp(rint(w / s), -(maxq+1), maxq); q = s * code
//   err  = ((w - q) - gh_i) / Hinv1[i][i]
//   w_j  = w_j - (err * Hinv1[i][j] + gh_j);   gh_j = gh_j - z_i * Hinv1[i][j]     (j >= i)
// so with identical inputs codes and errors are bit-identical to the reference's CPU loop.
// The atomic variant (:1238-1288) quantises the block start at once and solves
// Err * Hinv1 = W - Q - GHinv1 by forward substitution with the same row layout.
//
// Surrogate modes (:580-584, :1190-1199, :1360-1367): the first-order term used in place of
// gh is gh_eff = gh + beta_row * (W_cur - W_anchor), re-evaluated before every column, where
// W_anchor is the permuted weight before the first block, W_cur the live W1 (surrogate_online)
// or the block start (surrogate_block).  A fifth register array per row holds the anchor
// (online) or the constant difference W_block_start - W_anchor (block).
//
// k_trailing: W[:, i2:] -= Err Hinv[i1:i2, i2:] + (count GH[:, i2:] - (Z1 D) Hinv[i1:i2, i2:])
// and GH[:, i2:] -= Z1 Hinv[i1:i2, i2:], 64x64 output tiles, fp32 16x16x4 MFMA, K = count
// streamed through LDS in slabs of 32.  The Z terms are skipped when Z is identically zero.
// In the surrogate modes the GH[:, i2:] of the first term is GH + beta_row * (W - W_anchor)
// (outer refresh "surrogate_block", :1500-1511), the GH update itself is unchanged; in
// block_gd the whole W update is scaled by second_order_scale (:1546-1549).
#include <type_traits>

#include "rq_common.h"

namespace {

constexpr int QB_MAXB = 128;

// Compile-time loop: f(std::integral_constant<int, 0>) ... f(integral_constant<int, N - 1>).
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// Lanes per row in k_quant_block, and the broadcast of lane r of each 16-lane DPP row to the
// whole row (row_newbcast).
constexpr int QL = 16;
template <int R>
__device__ __forceinline__ float row_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + R, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

struct QBArgs {
  float* Wp;
  int64_t ldw;
  const float* Hinv;
  int C;
  const float* GH;
  const float* Z;
  int64_t ldgh;
  int R, R_s, i1, count, qmode;
  const float* scale;
  const int32_t* col_group;
  float* dyn_scale;
  float maxq;
  int sym, atomic;
  const int* z_nonzero;
  int16_t* codes;
  float* err;
  const float* anchor;
  int64_t lda;
  const float* beta;
  float sos;
};

// GM: 0 frozen, 1 surrogate_block, 2 surrogate_online, 3 frozen with every in-block update
// scaled by second_order_scale (block_gd, :1344-1349).  NS register slots per lane: lane t of
// a row holds columns t, t + 16, ..., t + 16 (NS - 1) of the block (NS = 8 for 128 columns).
template <int NS, int GM>
__global__ __launch_bounds__(256) void k_quant_block(QBArgs a) {
  constexpr int NB = QL * NS;             // widest block this instantiation takes
  // Hp[i][t][k] = Hinv1[i][16 k + t] (upper; zeros below the diagonal and past the block):
  // a lane reads its NS entries of row i as NS / 4 aligned 16-byte loads
  __shared__ __attribute__((aligned(16))) float Hp[NB][QL][NS];
  const int tid = threadIdx.x;
  const int t = tid & (QL - 1);
  const int sub = blockIdx.y;
  const int row_local = blockIdx.x * (256 / QL) + (tid / QL);
  const bool valid = row_local < a.R_s;
  const int row = sub * a.R_s + (valid ? row_local : 0);
  const int count = a.count, i1 = a.i1;
  const float* Hs = a.Hinv + (int64_t)sub * a.C * a.C;
  const bool use_gh = (*a.z_nonzero != 0);

  {
    // all NB * NB / 256 loads of a thread in flight at once: clamped (in-bounds) addresses,
    // the mask applied to the values
    constexpr int PER = NB * NB / 256;
    float v[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = tid + 256 * q, i = e / NB, j = e % NB;
      v[q] = Hs[(int64_t)(i1 + min(i, count - 1)) * a.C + (i1 + min(j, count - 1))];
    }
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = tid + 256 * q, i = e / NB, j = e % NB;
      Hp[i][j % QL][j / QL] = (i < count && j < count && j >= i) ? v[q] : 0.0f;
    }
  }

  constexpr bool SURR = (GM == 1 || GM == 2);
  float w[NS], gh[NS], zz[NS], sc[NS], xr[SURR ? NS : 1];
  const float brow = SURR ? a.beta[row] : 0.0f;
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const int col = QL * k + t;
    const bool in = valid && col < count;
    const int64_t off = (int64_t)row * a.ldw + i1 + col;
    w[k] = in ? a.Wp[off] : 0.0f;
    if constexpr (SURR) {
      const float wr = in ? a.anchor[(int64_t)row * a.lda + i1 + col] : 0.0f;
      xr[k] = (GM == 1) ? (w[k] - wr) : wr;
    }
    const int64_t og = (int64_t)row * a.ldgh + i1 + col;
    gh[k] = (in && use_gh) ? a.GH[og] : 0.0f;
    zz[k] = (in && use_gh) ? a.Z[og] : 0.0f;
    sc[k] = 0.0f;
    if (a.qmode == RQ_QMODE_STATIC && in) sc[k] = a.scale[(int64_t)a.col_group[i1 + col] * a.R + row];
  }
  // gh_eff of slot k from the current registers: gh + beta * (W_cur - W_anchor)
  auto geff = [&](int k) __attribute__((always_inline)) -> float {
    if constexpr (!SURR) return gh[k];
    const float dw = (GM == 1) ? xr[k] : (w[k] - xr[k]);
    return gh[k] + brow * dw;
  };
  const float lo = -(a.maxq + 1.0f), hi = a.maxq;
  float srow = 0.0f;
  if (a.qmode == RQ_QMODE_CHANNEL) {
    srow = a.scale[row];
  } else if (a.qmode == RQ_QMODE_DYNAMIC) {
    // find_params on the block start (gptq_plus_utils.py:1208-1209): per-row min/max over
    // the 16 lanes of the row (quad swaps, then rotations by 4 and 8 inside the row)
    float mn = __builtin_inff(), mx = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      if (QL * k + t < count) {
        mn = rq_nan_min(mn, w[k]);
        mx = rq_nan_max(mx, w[k]);
      }
    }
    mn = rq_nan_min(mn, dpp_mov<0xB1>(mn));
    mx = rq_nan_max(mx, dpp_mov<0xB1>(mx));
    mn = rq_nan_min(mn, dpp_mov<0x4E>(mn));
    mx = rq_nan_max(mx, dpp_mov<0x4E>(mx));
    mn = rq_nan_min(mn, dpp_mov<0x124>(mn));
    mx = rq_nan_max(mx, dpp_mov<0x124>(mx));
    mn = rq_nan_min(mn, dpp_mov<0x128>(mn));
    mx = rq_nan_max(mx, dpp_mov<0x128>(mx));
    float z;
    rq_params_from_minmax(mn, mx, a.maxq, a.sym, &srow, &z);
    if (valid && t == 0) a.dyn_scale[row] = srow;
  }
  __syncthreads();

  int16_t* crow = a.codes + (int64_t)row * a.C + i1;
  float* erow = a.err + (int64_t)row * count;
  // row i of the block for this lane: h[k] = Hinv1[i][16 k + t]
  auto hrow = [&](int i, float (&h)[NS]) __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < NS; k += 4) {
      const float4 v = *reinterpret_cast<const float4*>(&Hp[i][t][k]);
      h[k] = v.x;
      if (k + 1 < NS) h[k + 1] = v.y;
      if (k + 2 < NS) h[k + 2] = v.z;
      if (k + 3 < NS) h[k + 3] = v.w;
    }
  };

  if (a.atomic) {
    // Q1 = quant(W_block_start); res = W_block_start - Q1 - GHinv1   (:1243-1282)
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const int col = QL * k + t;
      const float s = (a.qmode == RQ_QMODE_STATIC) ? sc[k] : srow;
      const float code = rq_quant_code(w[k], s, lo, hi);
      const float q = s * code;
      if (valid && col < count) crow[col] = (code != code) ? RQ_CODE_NAN : (int16_t)code;
      const float ge = geff(k);
      w[k] = (w[k] - q) - ge;
    }
    // Err1 * Hinv1 = res, forward substitution (:1283-1288); column i = 16 m + r is owned by
    // lane r, slot m
    static_for<NS>([&](auto mc) __attribute__((always_inline)) {
      static_for<QL>([&](auto rc) __attribute__((always_inline)) {
        constexpr int m = decltype(mc)::value, r = decltype(rc)::value;
        const int i = QL * m + r;
        if (i < count) {
          float h[NS];
          hrow(i, h);
          const float e = row_bcast<r>(w[m] / h[m]);
          if (valid && t == r) erow[i] = e;
#pragma unroll
          for (int k = 0; k < NS; ++k) w[k] = w[k] - e * h[k];
        }
      });
    });
    return;
  }

  // column-serial loop (:1296-1367); column i = 16 m + r is quantised by lane r (slot m)
  auto column = [&](auto mc, auto rc, bool with_gh) __attribute__((always_inline)) {
    constexpr int m = decltype(mc)::value, r = decltype(rc)::value;
    const int i = QL * m + r;
    float h[NS];
    hrow(i, h);
    const float d = h[m];
    const float s = (a.qmode == RQ_QMODE_STATIC) ? sc[m] : srow;
    const float x = w[m];
    const float code = rq_quant_code(x, s, lo, hi);
    const float q = s * code;
    const float e = row_bcast<r>(((x - q) - geff(m)) / d);
    if (valid && t == r) {
      crow[i] = (code != code) ? RQ_CODE_NAN : (int16_t)code;
      erow[i] = e;
    }
    if constexpr (SURR) {
      const float zi = with_gh ? row_bcast<r>(zz[m]) : 0.0f;
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        const float ge = geff(k);
        const float upd = e * h[k];
        w[k] = w[k] - (upd + ge);
        gh[k] = gh[k] - zi * h[k];
      }
    } else if (with_gh) {
      const float zi = row_bcast<r>(zz[m]);
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        const float upd = e * h[k];
        if constexpr (GM == 3) w[k] = w[k] - a.sos * (upd + gh[k]);
        else w[k] = w[k] - (upd + gh[k]);
        gh[k] = gh[k] - zi * h[k];
      }
    } else {
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        if constexpr (GM == 3) w[k] = w[k] - a.sos * (e * h[k] + gh[k]);
        else w[k] = w[k] - (e * h[k] + gh[k]);
      }
    }
  };
  auto all_columns = [&](bool with_gh) __attribute__((always_inline)) {
    static_for<NS>([&](auto mc) __attribute__((always_inline)) {
      static_for<QL>([&](auto rc) __attribute__((always_inline)) {
        if (QL * decltype(mc)::value + decltype(rc)::value < count) column(mc, rc, with_gh);
      });
    });
  };
  if (use_gh) all_columns(true);
  else all_columns(false);
}

// ---------------------------------------------------------------------------------------
struct TrArgs {
  float* Wp;
  int64_t ldw;
  float* GH;
  const float* Z;
  int64_t ldgh;
  const float* Hinv;
  int C, R, R_s, i1, count;
  const float* err;
  const int* z_nonzero;
  int gmode;
  const float* anchor;
  int64_t lda;
  const float* beta;
  float sos;
};

constexpr int TKS = 32;  // K slab
constexpr int TPAD = 4;

__global__ __launch_bounds__(256) void k_trailing(TrArgs a) {
  __shared__ float Es[TKS][64 + TPAD];
  __shared__ float Zs[TKS][64 + TPAD];
  __shared__ float Hs[TKS][64 + TPAD];
  const int i2 = a.i1 + a.count;
  const int sub = blockIdx.z;
  const int rl0 = blockIdx.y * 64;
  const int c0 = i2 + blockIdx.x * 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const bool use_z = (*a.z_nonzero != 0);
  const float* Hsub = a.Hinv + (int64_t)sub * a.C * a.C;
  const int rbase = sub * a.R_s;

  floatx4 acc1[2][2], acc2[2][2], acc3[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc1[x][y][e] = acc2[x][y][e] = acc3[x][y][e] = 0.0f;

  for (int k0 = 0; k0 < a.count; k0 += TKS) {
    __syncthreads();
    // err / Z slabs: 64 rows x 32 k, stored k-major; H slab: 32 k x 64 cols
    for (int e = tid; e < 64 * TKS; e += 256) {
      const int rr = e / TKS, kk = e % TKS;
      const int rl = rl0 + rr, k = k0 + kk;
      const bool in = rl < a.R_s && k < a.count;
      Es[kk][rr] = in ? a.err[(int64_t)(rbase + rl) * a.count + k] : 0.0f;
      if (use_z) Zs[kk][rr] = in ? a.Z[(int64_t)(rbase + rl) * a.ldgh + a.i1 + k] : 0.0f;
    }
    for (int e = tid; e < TKS * 64; e += 256) {
      const int kk = e / 64, cc = e % 64;
      const int k = k0 + kk, c = c0 + cc;
      Hs[kk][cc] = (k < a.count && c < a.C) ? Hsub[(int64_t)(a.i1 + k) * a.C + c] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < TKS / 4; ++kk) {
      const int k = kk * 4 + (lane >> 4);
      const float b0 = Hs[k][wc * 32 + (lane & 15)];
      const float b1 = Hs[k][wc * 32 + 16 + (lane & 15)];
      const float e0 = Es[k][wr * 32 + (lane & 15)];
      const float e1 = Es[k][wr * 32 + 16 + (lane & 15)];
      acc1[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(e0, b0, acc1[0][0], 0, 0, 0);
      acc1[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(e0, b1, acc1[0][1], 0, 0, 0);
      acc1[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(e1, b0, acc1[1][0], 0, 0, 0);
      acc1[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(e1, b1, acc1[1][1], 0, 0, 0);
      if (use_z) {
        const float dk = (float)(a.count - 1 - (k0 + k));
        const float z0 = Zs[k][wr * 32 + (lane & 15)];
        const float z1 = Zs[k][wr * 32 + 16 + (lane & 15)];
        const float zd0 = z0 * dk, zd1 = z1 * dk;
        acc2[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(zd0, b0, acc2[0][0], 0, 0, 0);
        acc2[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(zd0, b1, acc2[0][1], 0, 0, 0);
        acc2[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(zd1, b0, acc2[1][0], 0, 0, 0);
        acc2[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(zd1, b1, acc2[1][1], 0, 0, 0);
        acc3[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(z0, b0, acc3[0][0], 0, 0, 0);
        acc3[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(z0, b1, acc3[0][1], 0, 0, 0);
        acc3[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(z1, b0, acc3[1][0], 0, 0, 0);
        acc3[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(z1, b1, acc3[1][1], 0, 0, 0);
      }
    }
  }

  const float cnt = (float)a.count;
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int rl = rl0 + wr * 32 + x * 16 + 4 * (lane >> 4) + e;
        const int c = c0 + wc * 32 + y * 16 + (lane & 15);
        if (rl < a.R_s && c < a.C) {
          const int64_t ow = (int64_t)(rbase + rl) * a.ldw + c;
          if (a.gmode == 1 || a.gmode == 2) {
            const float wv = a.Wp[ow];
            const float g = use_z ? a.GH[(int64_t)(rbase + rl) * a.ldgh + c] : 0.0f;
            const float dw = wv - a.anchor[(int64_t)(rbase + rl) * a.lda + c];
            const float geff = g + a.beta[rbase + rl] * dw;
            const float gupd = cnt * geff - acc2[x][y][e];
            a.Wp[ow] = wv - (acc1[x][y][e] + gupd);
            if (use_z) a.GH[(int64_t)(rbase + rl) * a.ldgh + c] = g - acc3[x][y][e];
          } else if (use_z) {
            const int64_t og = (int64_t)(rbase + rl) * a.ldgh + c;
            const float g = a.GH[og];
            const float gupd = cnt * g - acc2[x][y][e];
            const float tot = acc1[x][y][e] + gupd;
            a.Wp[ow] = a.Wp[ow] - (a.gmode == 3 ? a.sos * tot : tot);
            a.GH[og] = g - acc3[x][y][e];
          } else {
            const float tot = acc1[x][y][e];
            a.Wp[ow] = a.Wp[ow] - (a.gmode == 3 ? a.sos * tot : tot);
          }
        }
      }
}

}  // namespace

extern "C" int rq_quant_block(float* Wp, int64_t ldw, const float* Hinv_all, int C, const float* GH,
                              const float* Z, int64_t ldgh, int R, int R_s, int i1, int count,
                              int qmode, const float* scale, const int32_t* col_group,
                              float* dyn_scale, int maxq, int sym, int atomic,
                              const int* z_nonzero, int16_t* codes, float* err, int gmode,
                              const float* anchor, int64_t ld_anchor, const float* beta,
                              double second_order_scale, void* stream) {
  if (!Wp || !Hinv_all || !GH || !Z || !z_nonzero || !codes || !err) return RQ_EINVAL;
  if (gmode < 0 || gmode > 3) return RQ_EINVAL;
  if ((gmode == 1 || gmode == 2) && (!anchor || !beta || ld_anchor < C)) return RQ_EINVAL;
  if (R <= 0 || R_s <= 0 || R % R_s != 0 || C <= 0 || ldw < C || ldgh < C) return RQ_EINVAL;
  if (count <= 0 || count > QB_MAXB || i1 < 0 || i1 + count > C || maxq <= 0) return RQ_EINVAL;
  if (qmode == RQ_QMODE_CHANNEL && !scale) return RQ_EINVAL;
  if (qmode == RQ_QMODE_STATIC && (!scale || !col_group)) return RQ_EINVAL;
  if (qmode == RQ_QMODE_DYNAMIC && !dyn_scale) return RQ_EINVAL;
  if (qmode < 0 || qmode > 2) return RQ_EINVAL;
  QBArgs a{Wp, ldw, Hinv_all, C, GH, Z, ldgh, R, R_s, i1, count, qmode, scale, col_group,
           dyn_scale, (float)maxq, sym, atomic, z_nonzero, codes, err, anchor, ld_anchor, beta,
           (float)second_order_scale};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((R_s + 256 / QL - 1) / (256 / QL), R / R_s), block(256);
  const bool small = count <= 2 * QL;
  switch (gmode) {
    case 0:
      if (small) hipLaunchKernelGGL((k_quant_block<2, 0>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((k_quant_block<8, 0>), grid, block, 0, s, a);
      break;
    case 1:
      if (small) hipLaunchKernelGGL((k_quant_block<2, 1>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((k_quant_block<8, 1>), grid, block, 0, s, a);
      break;
    case 2:
      if (small) hipLaunchKernelGGL((k_quant_block<2, 2>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((k_quant_block<8, 2>), grid, block, 0, s, a);
      break;
    default:
      if (small) hipLaunchKernelGGL((k_quant_block<2, 3>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((k_quant_block<8, 3>), grid, block, 0, s, a);
  }
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}

extern "C" int rq_trailing_update(float* Wp, int64_t ldw, float* GH, const float* Z, int64_t ldgh,
                                  const float* Hinv_all, int C, int R, int R_s, int i1, int count,
                                  const float* err, const int* z_nonzero, int gmode,
                                  const float* anchor, int64_t ld_anchor, const float* beta,
                                  double second_order_scale, void* stream) {
  if (!Wp || !GH || !Z || !Hinv_all || !err || !z_nonzero) return RQ_EINVAL;
  if (gmode < 0 || gmode > 3) return RQ_EINVAL;
  if ((gmode == 1 || gmode == 2) && (!anchor || !beta || ld_anchor < C)) return RQ_EINVAL;
  if (R <= 0 || R_s <= 0 || R % R_s != 0 || C <= 0 || ldw < C || ldgh < C) return RQ_EINVAL;
  if (count <= 0 || i1 < 0 || i1 + count > C) return RQ_EINVAL;
  const int i2 = i1 + count;
  if (i2 >= C) return RQ_OK;
  TrArgs a{Wp, ldw, GH, Z, ldgh, Hinv_all, C, R, R_s, i1, count, err, z_nonzero, gmode,
           anchor, ld_anchor, beta, (float)second_order_scale};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((C - i2 + 63) / 64, (R_s + 63) / 64, R / R_s), block(256);
  hipLaunchKernelGGL(k_trailing, grid, block, 0, s, a);
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}
