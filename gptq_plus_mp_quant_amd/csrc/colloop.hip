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
// k_trailing_w (Z identically zero, frozen / block_gd): W[:, i2:] -= Err Hinv[i1:i2, i2:] with
// the product formed as a k-ordered fused multiply-add chain on the matrix cores, bit-identical
// to the reference's CPU matmul (see the kernel).  Otherwise k_trailing_z:
// W[:, i2:] -= Err Hinv[i1:i2, i2:] + (count GH[:, i2:] - (Z1 D) Hinv[i1:i2, i2:]) and
// GH[:, i2:] -= Z1 Hinv[i1:i2, i2:], the three products formed the same way, so with equal
// inputs W and GH are the reference's bit for bit.  In the surrogate modes the GH[:, i2:] of
// the first term is GH + beta_row * (W - W_anchor) (outer refresh "surrogate_block",
// :1500-1511), the GH update itself is unchanged; in block_gd the whole W update is scaled by
// second_order_scale (:1546-1549).  k_trailing (fp32 16x16x4 MFMA, 64x64 tiles) takes the
// shapes those two cannot (a block width that is not a multiple of 8, unaligned operands).
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
  // Look-ahead launch (k_block_lookahead): the previous block's update of this block's
  // columns, applied by each workgroup to its own rows before the column loop; zero_terms: Z
  // (hence GH) is identically zero, z_nonzero is not read.
  const float* near_err;      // err of the previous block [R, near_count], or NULL
  int near_i1, near_count;
  int zero_terms;
};

// Bytes of LDS the column loop uses: the block of Hinv ([16 NS][16][NS] floats), and in a
// look-ahead launch the previous block's rows of Hinv ([QB_MAXB][16][NS], the same buffer)
// and err of the workgroup's 16 rows after it.
template <int NS>
constexpr int qb_hbytes(bool near) {
  return (near ? QB_MAXB : QL * NS) * QL * NS * 4;
}
template <int NS>
constexpr int qb_lds_bytes(bool near) {
  return qb_hbytes<NS>(near) + (near ? (256 / QL) * QB_MAXB * 4 : 0);
}

// GM: 0 frozen, 1 surrogate_block, 2 surrogate_online, 3 frozen with every in-block update
// scaled by second_order_scale (block_gd, :1344-1349).  NS register slots per lane: lane t of
// a row holds columns t, t + 16, ..., t + 16 (NS - 1) of the block (NS = 8 for 128 columns).
template <int NS, int GM>
__device__ __forceinline__ void quant_block_body(const QBArgs& a, int bx, int by, uint8_t* lds) {
  constexpr int NB = QL * NS;             // widest block this instantiation takes
  // Hp[i][t][k] = Hinv1[i][16 k + t] (upper; zeros below the diagonal and past the block):
  // a lane reads its NS entries of row i as NS / 4 aligned 16-byte loads
  float (*Hp)[QL][NS] = reinterpret_cast<float (*)[QL][NS]>(lds);
  const int tid = threadIdx.x;
  const int t = tid & (QL - 1);
  const int sub = by;
  const int rloc = tid / QL;
  const int row_local = bx * (256 / QL) + rloc;
  const bool valid = row_local < a.R_s;
  const int row = sub * a.R_s + (valid ? row_local : 0);
  const int count = a.count, i1 = a.i1;
  const float* Hs = a.Hinv + (int64_t)sub * a.C * a.C;
  const bool use_gh = !a.zero_terms && (*a.z_nonzero != 0);

  // Look-ahead launch: W[r, i1 + c] -= sum_k err_prev[r, k] Hinv[p1 + k, i1 + c] for this
  // workgroup's rows, formed like rq_trailing_update (a sequential fused multiply-add chain in k
  // from 0, then one subtraction: the CPU matmul's order), and written back to Wp.  The
  // previous block's rows of Hinv go through the same LDS as Hp (Hoff[k][t][s] =
  // Hinv[p1 + k][i1 + 16 s + t]), the err rows after it.
  float wn[NS];                         // the block's weights after the look-ahead update
  if (a.near_err) {
    const int pc = a.near_count, p1 = a.near_i1;
    float* Ep = reinterpret_cast<float*>(lds + qb_hbytes<NS>(true));   // [16][QB_MAXB]
    constexpr int PER = QB_MAXB * NB / 256;
    float v[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = tid + 256 * q, i = e / NB, j = e % NB;
      v[q] = Hs[(int64_t)(p1 + min(i, pc - 1)) * a.C + (i1 + min(j, count - 1))];
    }
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = tid + 256 * q, i = e / NB, j = e % NB;
      Hp[i][j % QL][j / QL] = (i < pc && j < count) ? v[q] : 0.0f;
    }
    for (int e = tid; e < (256 / QL) * pc; e += 256) {
      const int rl = e / pc, kk = e % pc;
      const int rr = bx * (256 / QL) + rl;
      Ep[rl * QB_MAXB + kk] = (rr < a.R_s) ? a.near_err[(int64_t)(sub * a.R_s + rr) * pc + kk] : 0.0f;
    }
    __syncthreads();
    float acc[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) acc[k] = 0.0f;
    const float* er = Ep + rloc * QB_MAXB;
    for (int kk = 0; kk < pc; ++kk) {
      const float e = er[kk];
#pragma unroll
      for (int k = 0; k < NS; k += 4) {
        const float4 h = *reinterpret_cast<const float4*>(&Hp[kk][t][k]);
        acc[k] = __builtin_fmaf(e, h.x, acc[k]);
        if (k + 1 < NS) acc[k + 1] = __builtin_fmaf(e, h.y, acc[k + 1]);
        if (k + 2 < NS) acc[k + 2] = __builtin_fmaf(e, h.z, acc[k + 2]);
        if (k + 3 < NS) acc[k + 3] = __builtin_fmaf(e, h.w, acc[k + 3]);
      }
    }
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const int col = QL * k + t;
      const bool in = valid && col < count;
      float* wp = a.Wp + (int64_t)row * a.ldw + i1 + col;
      wn[k] = in ? *wp - acc[k] : 0.0f;
      if (in) *wp = wn[k];
    }
    __syncthreads();                  // Hp is refilled below
  }

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
    w[k] = a.near_err ? wn[k] : (in ? a.Wp[off] : 0.0f);
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
    // lane r, slot m.  The operations are those of the CPU triangular solve (MKL strsm, which
    // for blocks of up to 32 columns is this unblocked substitution): e_i = c_i * (1 / Hinv1[i][i])
    // and c_k = fma(-e_i, Hinv1[i][k], c_k), applied to c_k for i = 0, 1, ... in order.
    static_for<NS>([&](auto mc) __attribute__((always_inline)) {
      static_for<QL>([&](auto rc) __attribute__((always_inline)) {
        constexpr int m = decltype(mc)::value, r = decltype(rc)::value;
        const int i = QL * m + r;
        if (i < count) {
          float h[NS];
          hrow(i, h);
          const float e = row_bcast<r>(w[m] * (1.0f / h[m]));
          if (valid && t == r) erow[i] = e;
#pragma unroll
          for (int k = 0; k < NS; ++k) w[k] = __builtin_fmaf(-e, h[k], w[k]);
        }
      });
    });
    return;
  }

  // column-serial loop (:1296-1367); column i = 16 m + r is quantised by lane r (slot m).  The
  // updates of a column reach the slots k >= m only: slots below hold finished columns, which
  // the reference no longer updates either (W1[:, i:]).  Each lane keeps the codes and errors
  // of its own slots in registers and stores them after the loop.
  float ccode[NS], cerr[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    ccode[k] = 0.0f;
    cerr[k] = 0.0f;
  }
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
    ccode[m] = (t == r) ? code : ccode[m];
    cerr[m] = (t == r) ? e : cerr[m];
    if constexpr (SURR) {
      const float zi = with_gh ? row_bcast<r>(zz[m]) : 0.0f;
#pragma unroll
      for (int k = m; k < NS; ++k) {
        const float ge = geff(k);
        const float upd = e * h[k];
        w[k] = w[k] - (upd + ge);
        gh[k] = gh[k] - zi * h[k];
      }
    } else if (with_gh) {
      const float zi = row_bcast<r>(zz[m]);
#pragma unroll
      for (int k = m; k < NS; ++k) {
        const float upd = e * h[k];
        if constexpr (GM == 3) w[k] = w[k] - a.sos * (upd + gh[k]);
        else w[k] = w[k] - (upd + gh[k]);
        gh[k] = gh[k] - zi * h[k];
      }
    } else {
#pragma unroll
      for (int k = m; k < NS; ++k) {
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
  if (valid) {
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const int col = QL * k + t;
      if (col < count) {
        crow[col] = (ccode[k] != ccode[k]) ? RQ_CODE_NAN : (int16_t)ccode[k];
        erow[col] = cerr[k];
      }
    }
  }
}

template <int NS, int GM>
__global__ __launch_bounds__(256) void k_quant_block(QBArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[qb_lds_bytes<NS>(false)];
  quant_block_body<NS, GM>(a, blockIdx.x, blockIdx.y, lds);
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

// ---------------------------------------------------------------------------------------
// k_trailing_w: the frozen-mode outer update when Z is identically zero (then GH is zero too):
//   W[r, i2:] -= f * sum_k err[r, k] Hinv_s[i1 + k, i2:]       (f = 1, or second_order_scale)
// The sum is formed like the reference's CPU matmul, a sequential fused multiply-add chain
// c = fma(err[r, k], Hinv[k, c], c) for k = 0, 1, ..., count-1 starting from 0, so W is
// bit-identical to `W - Err1 @ Hinv[i1:i2, i2:]` on CPU: every step is one
// v_mfma_f32_32x32x1_2b_f32 (a 32x32 outer product per block, k = 1), which rounds exactly like
// one fmaf per output, issued in k order.
// 128 x 128 output tiles inside one subgroup, 4 waves of 64 x 64; per k a wave issues two of
// them (column halves 0-31 and 32-63; in each, block b takes rows 32b .. 32b+31 of the wave, so
// lane l supplies err of wave row l and Hinv of column l % 32 of the half).  K advances 8 at a
// time through a ring of TSTAGES LDS stages (separate __shared__ arrays, the loop unrolled by
// TSTAGES so stage indices are compile-time constants), filled by direct global -> LDS loads
// (16 bytes per lane) issued TSTAGES-1 steps ahead; one barrier per step.  Per stage and wave:
// one 1 KB chunk of err (32 rows x 8 k; lane L fetches row L/2, k quad (L%2) ^ ((row/8)%2), so
// a lane's two 16-byte reads of its row are conflict-free) and one of Hinv (2 k-rows x 128
// columns, chunks 64 bytes apart; both halves of the wave read the same word: a broadcast).
constexpr int TT = 128;
constexpr int TSTAGES = 4;
constexpr int TCH = 1024;
constexpr int THROW = TCH + 64;          // Hinv chunk stride in a stage
constexpr int TA_BYTES = 4 * TCH;
constexpr int TSTAGE = TA_BYTES + 4 * THROW;

typedef float floatx32 __attribute__((ext_vector_type(32)));

struct TwArgs {
  float* Wp;
  int64_t ldw;
  const float* Hinv;
  int C, R_s, i1, count;
  const float* err;
  float f;               // 1, or second_order_scale (RQ_GMODE_BLOCK_GD)
  int nrt, nct;          // row tiles per subgroup, column tiles
  int total;             // nrt * nct * subgroups
  int cbeg;              // first updated column (i1 + count; later in a look-ahead launch)
};

struct TStages {
  uint8_t* s[TSTAGES];
};

__device__ __forceinline__ void lds_dma16(const void* g, uint8_t* l) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)l, 16, 0, 0);
}

// s_waitcnt with only the vector-memory counter limited (gfx9 encoding).
#define TWAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

struct TwTile {
  const float* srcA;
  const float* srcB;
  int wave, wc, aoff0, aoff1, boff, nk;
  int64_t ldh;
  floatx32 acc[2];

  __device__ __forceinline__ void stage(uint8_t* st, int kt) {
    lds_dma16(srcA + kt * 8, st + wave * TCH);
    lds_dma16(srcB + (int64_t)kt * 8 * ldh, st + TA_BYTES + wave * THROW);
  }
  // Step kt: wait for this wave's 2 staging loads of kt (the TSTAGES-2 later steps may be in
  // flight), meet the other waves (their parts are in LDS, and every read of the FILL stage,
  // done in step kt-1, is over), refill FILL with step kt+TSTAGES-1, then k = 8 kt .. 8 kt + 7.
  template <int CUR, int FILL>
  __device__ __forceinline__ void step(const TStages& L, int kt) {
    TWAIT_VM(2 * (TSTAGES - 2));
    RQ_STAGE_BARRIER();
    stage(L.s[FILL], min(kt + TSTAGES - 1, nk - 1));
    const uint8_t* st = L.s[CUR];
    const float4 a0 = *reinterpret_cast<const float4*>(st + aoff0);   // k 0..3 of this lane's row
    const float4 a1 = *reinterpret_cast<const float4*>(st + aoff1);   // k 4..7
    const float av[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    float bv[8][2];
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        bv[k][h] = *reinterpret_cast<const float*>(st + TA_BYTES + (k >> 1) * THROW + (k & 1) * 512 +
                                                    boff + 128 * h);
    // all reads of the step issued before its MFMAs (otherwise the scheduler reuses one
    // register pair for every Hinv read and each MFMA pair waits for an LDS round trip)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int h = 0; h < 2; ++h) acc[h] = __builtin_amdgcn_mfma_f32_32x32x1f32(av[k], bv[k][h], acc[h], 0, 0, 0);
  }
};

__device__ __forceinline__ void trailing_w_body(const TwArgs& a, int b, const TStages& L) {
  // XCD-aware order: each XCD takes a contiguous range of tiles (row tile fastest), so the
  // tiles of one Hinv column strip meet in one L2.
  const int per = a.total / 8, rem8 = a.total % 8;
  const int xcd = b % 8, idx = b / 8;
  const int t = (xcd < rem8) ? xcd * (per + 1) + idx : rem8 * (per + 1) + (xcd - rem8) * per + idx;
  if (t >= a.total) return;
  const int per_sub = a.nrt * a.nct;
  const int sub = t / per_sub, u = t % per_sub;
  const int ct = u / a.nrt, rt = u % a.nrt;
  const int rl0 = rt * TT, c0 = a.cbeg + ct * TT;
  const int64_t rbase = (int64_t)sub * a.R_s;

  TwTile w;
  const int tid = threadIdx.x, lane = tid & 63;
  w.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = w.wave >> 1;
  w.wc = w.wave & 1;
  w.nk = a.count / 8;
  w.ldh = a.C;
  {
    // staging sources: err chunk `wave` (rows 32 wave .. +31 of the tile), Hinv k-rows
    // 2 wave, 2 wave + 1 (columns clamped to a whole in-bounds quad)
    const int rho = lane >> 1, q = (lane & 1) ^ ((rho >> 3) & 1);
    const int rl = min(rl0 + 32 * w.wave + rho, a.R_s - 1);
    w.srcA = a.err + (rbase + rl) * a.count + 4 * q;
    const int kr = 2 * w.wave + (lane >> 5);
    const int c = min(c0 + 4 * (lane & 31), a.C - 4);
    w.srcB = a.Hinv + (int64_t)sub * a.C * a.C + (int64_t)(a.i1 + kr) * a.C + c;
  }
  // err of this lane: wave row `lane` = tile row 64 wr + lane, in chunk 2 wr + lane / 32 at
  // in-chunk row rho = lane % 32; k quad q sits at slot 2 rho + (q ^ ((rho / 8) % 2))
  {
    const int rho = lane & 31, sw = (rho >> 3) & 1;
    const int base = (2 * wr + (lane >> 5)) * TCH + 32 * rho;
    w.aoff0 = base + 16 * (0 ^ sw);
    w.aoff1 = base + 16 * (1 ^ sw);
  }
  // Hinv of this lane: column 64 wc + 32 h + lane % 32 of the tile
  w.boff = 4 * (64 * w.wc + (lane & 31));
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 32; ++e) w.acc[h][e] = 0.0f;

  // This lane's 64 outputs of W (clamped in-bounds addresses), loaded before the staging so
  // their latency overlaps the first stage's: output e of half h is wave row
  // 32 (e / 16) + 8 ((e % 16) / 4) + 4 (lane / 32) + e % 4, wave column 32 h + lane % 32.
  const int rw0 = rl0 + 64 * wr + 4 * (lane >> 5), cw0 = c0 + 64 * w.wc + (lane & 31);
  float wv[2][32];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const int rl = min(rw0 + 32 * (e / 16) + 8 * ((e % 16) / 4) + (e % 4), a.R_s - 1);
      wv[h][e] = a.Wp[(rbase + rl) * a.ldw + min(cw0 + 32 * h, a.C - 1)];
    }

  static_assert(TSTAGES == 4, "unrolled stage schedule");
#pragma unroll
  for (int s = 0; s < TSTAGES - 1; ++s) w.stage(L.s[s], min(s, w.nk - 1));
  int kt = 0;
  for (; kt + 4 <= w.nk; kt += 4) {
    w.step<0, 3>(L, kt);
    w.step<1, 0>(L, kt + 1);
    w.step<2, 1>(L, kt + 2);
    w.step<3, 2>(L, kt + 3);
  }
  const int rem = w.nk - kt;
  if (rem > 0) w.step<0, 3>(L, kt);
  if (rem > 1) w.step<1, 0>(L, kt + 1);
  if (rem > 2) w.step<2, 1>(L, kt + 2);
  TWAIT_VM(0);   // no staging in flight when the workgroup ends

  // W - tot, or W - f * tot (block_gd), into the prefetched outputs.
  const bool full = (rl0 + TT <= a.R_s) && (c0 + TT <= a.C);
  const bool scaled = a.f != 1.0f;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const int rl = rw0 + 32 * (e / 16) + 8 * ((e % 16) / 4) + (e % 4), c = cw0 + 32 * h;
      const float tot = w.acc[h][e];
      const float v = wv[h][e] - (scaled ? a.f * tot : tot);
      if (full || (rl < a.R_s && c < a.C)) a.Wp[(rbase + rl) * a.ldw + c] = v;
    }
}

__global__ __launch_bounds__(256, 2) void k_trailing_w(TwArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds0[TSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds1[TSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds2[TSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds3[TSTAGE];
  const TStages L{{lds0, lds1, lds2, lds3}};
  trailing_w_body(a, blockIdx.x, L);
}

// One launch per block k of the frozen column loop with Z identically zero: workgroups
// [0, nq) quantise block k+1 (each first applies block k's update to its own rows of block
// k+1's columns), the others update the columns past block k+1 with block k's err
// (k_trailing_w's tiles).  The two parts touch disjoint columns and different err buffers,
// so block k+1's column loop runs while block k's wide update does.  The quantising
// workgroups come first in the grid, so they are dispatched first.
template <int NS>
__global__ __launch_bounds__(256, 2) void k_block_lookahead(QBArgs q, TwArgs w, int nqx, int nq) {
  constexpr int QBYTES = qb_lds_bytes<NS>(true);
  constexpr int LBYTES = QBYTES > TSTAGES * TSTAGE ? QBYTES : TSTAGES * TSTAGE;
  __shared__ __attribute__((aligned(16))) uint8_t lds[LBYTES];
  const int b = blockIdx.x;
  if (b < nq) {
    quant_block_body<NS, 0>(q, b % nqx, b / nqx, lds);
    return;
  }
  const TStages L{{lds, lds + TSTAGE, lds + 2 * TSTAGE, lds + 3 * TSTAGE}};
  trailing_w_body(w, b - nq, L);
}

// ---------------------------------------------------------------------------------------
// k_trailing_z: the outer update with the GPTQ+ terms (gptq_plus_utils.py:1500-1570), every
// product a k-ordered fused multiply-add chain like the reference's CPU matmuls (K = count):
//   second = Err1 @ Hinv[i1:i2, i2:]
//   zd     = (Z1 * D) @ Hinv[i1:i2, i2:]      (torch's einsum("ij,j,jk->ik") on CPU is exactly
//                                               this: the elementwise product, then the matmul)
//   zz     = Z1 @ Hinv[i1:i2, i2:]
//   W  -= second + (count * gh_eff - zd)      (block_gd: W -= sos * (...))
//   GH -= zz
// with gh_eff = GH, or GH + beta_r * (W - W_anchor) in the surrogate modes.  Each step is one
// v_mfma_f32_32x32x1_2b_f32 per chain, so with equal inputs W and GH equal the reference's.
// 64 x 128 output tiles: the 4 waves share the tile's 64 rows and take 32 columns each (three
// 64 x 32 accumulators per wave).  The K ring is k_trailing_w's; per stage waves 0-1 fetch the
// Err1 chunks of the two 32-row halves, waves 2-3 the Z1 chunks, every wave two Hinv k-rows.
struct TzArgs {
  float* Wp;
  int64_t ldw;
  float* GH;
  const float* Z;
  int64_t ldgh;
  const float* Hinv;
  int C, R_s, i1, count;
  const float* err;
  int gmode;
  const float* anchor;
  int64_t lda;
  const float* beta;
  float sos;
  int nrt, nct, total;
};

constexpr int TZR = 64;    // tile rows
constexpr int TZC = 128;   // tile columns

struct TzTile {
  const float* srcA;
  const float* srcB;
  int wave, eoff0, eoff1, boff, nk, count;
  int64_t ldh;
  floatx32 accE, accD, accZ;

  __device__ __forceinline__ void stage(uint8_t* st, int kt) {
    lds_dma16(srcA + kt * 8, st + wave * TCH);
    lds_dma16(srcB + (int64_t)kt * 8 * ldh, st + TA_BYTES + wave * THROW);
  }
  template <int CUR, int FILL>
  __device__ __forceinline__ void step(const TStages& L, int kt) {
    TWAIT_VM(2 * (TSTAGES - 2));
    RQ_STAGE_BARRIER();
    stage(L.s[FILL], min(kt + TSTAGES - 1, nk - 1));
    const uint8_t* st = L.s[CUR];
    const float4 e0 = *reinterpret_cast<const float4*>(st + eoff0);
    const float4 e1 = *reinterpret_cast<const float4*>(st + eoff1);
    const float4 z0 = *reinterpret_cast<const float4*>(st + 2 * TCH + eoff0);
    const float4 z1 = *reinterpret_cast<const float4*>(st + 2 * TCH + eoff1);
    const float ev[8] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w};
    const float zv[8] = {z0.x, z0.y, z0.z, z0.w, z1.x, z1.y, z1.z, z1.w};
    float bv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      bv[k] = *reinterpret_cast<const float*>(st + TA_BYTES + (k >> 1) * THROW + (k & 1) * 512 + boff);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float zd = zv[k] * (float)(count - 1 - (8 * kt + k));   // (Z1 * D)[r, k], one rounding
      accE = __builtin_amdgcn_mfma_f32_32x32x1f32(ev[k], bv[k], accE, 0, 0, 0);
      accD = __builtin_amdgcn_mfma_f32_32x32x1f32(zd, bv[k], accD, 0, 0, 0);
      accZ = __builtin_amdgcn_mfma_f32_32x32x1f32(zv[k], bv[k], accZ, 0, 0, 0);
    }
  }
};

template <bool SURR>
__global__ __launch_bounds__(256, 2) void k_trailing_z(TzArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds0[TSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds1[TSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds2[TSTAGE];
  __shared__ __attribute__((aligned(16))) uint8_t lds3[TSTAGE];
  const TStages L{{lds0, lds1, lds2, lds3}};
  const int b = blockIdx.x;
  const int per = a.total / 8, rem8 = a.total % 8;
  const int xcd = b % 8, idx = b / 8;
  const int t = (xcd < rem8) ? xcd * (per + 1) + idx : rem8 * (per + 1) + (xcd - rem8) * per + idx;
  if (t >= a.total) return;
  const int per_sub = a.nrt * a.nct;
  const int sub = t / per_sub, u = t % per_sub;
  const int ct = u / a.nrt, rt = u % a.nrt;
  const int i2 = a.i1 + a.count;
  const int rl0 = rt * TZR, c0 = i2 + ct * TZC;
  const int64_t rbase = (int64_t)sub * a.R_s;
  const int tid = threadIdx.x, lane = tid & 63;

  TzTile w;
  w.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  w.nk = a.count / 8;
  w.count = a.count;
  w.ldh = a.C;
  {
    // staging sources: waves 0-1 Err1 rows 32 w .. +31 of the tile, waves 2-3 Z1 rows
    // 32 (w - 2) .. +31 (lane L: row L / 2, k quad (L % 2) ^ ((row / 8) % 2)); every wave the
    // Hinv k-rows 2 w, 2 w + 1 (columns clamped to a whole in-bounds quad)
    const int rho = lane >> 1, q = (lane & 1) ^ ((rho >> 3) & 1);
    const int rl = min(rl0 + 32 * (w.wave & 1) + rho, a.R_s - 1);
    w.srcA = (w.wave < 2) ? a.err + (rbase + rl) * a.count + 4 * q
                          : a.Z + (rbase + rl) * a.ldgh + a.i1 + 4 * q;
    const int kr = 2 * w.wave + (lane >> 5);
    const int c = min(c0 + 4 * (lane & 31), a.C - 4);
    w.srcB = a.Hinv + (int64_t)sub * a.C * a.C + (int64_t)(a.i1 + kr) * a.C + c;
  }
  {
    // this lane's row is tile row `lane`: Err1 chunk lane / 32, Z1 chunk 2 + lane / 32
    const int rho = lane & 31, sw = (rho >> 3) & 1;
    const int base = (lane >> 5) * TCH + 32 * rho;
    w.eoff0 = base + 16 * (0 ^ sw);
    w.eoff1 = base + 16 * (1 ^ sw);
  }
  w.boff = 4 * (32 * w.wave + (lane & 31));
#pragma unroll
  for (int e = 0; e < 32; ++e) w.accE[e] = w.accD[e] = w.accZ[e] = 0.0f;

  // this lane's 32 outputs: tile row 32 (e / 16) + 8 ((e % 16) / 4) + 4 (lane / 32) + e % 4,
  // column 32 wave + lane % 32; W and GH loaded before the K loop (the surrogate modes' anchor
  // after it, to stay within the register budget)
  const int rw0 = rl0 + 4 * (lane >> 5), cw = c0 + 32 * w.wave + (lane & 31);
  float wv[32], gv[32];
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const int rl = min(rw0 + 32 * (e / 16) + 8 * ((e % 16) / 4) + (e % 4), a.R_s - 1);
    const int c = min(cw, a.C - 1);
    wv[e] = a.Wp[(rbase + rl) * a.ldw + c];
    gv[e] = a.GH[(rbase + rl) * a.ldgh + c];
  }

  static_assert(TSTAGES == 4, "unrolled stage schedule");
#pragma unroll
  for (int s = 0; s < TSTAGES - 1; ++s) w.stage(L.s[s], min(s, w.nk - 1));
  int kt = 0;
  for (; kt + 4 <= w.nk; kt += 4) {
    w.step<0, 3>(L, kt);
    w.step<1, 0>(L, kt + 1);
    w.step<2, 1>(L, kt + 2);
    w.step<3, 2>(L, kt + 3);
  }
  const int rem = w.nk - kt;
  if (rem > 0) w.step<0, 3>(L, kt);
  if (rem > 1) w.step<1, 0>(L, kt + 1);
  if (rem > 2) w.step<2, 1>(L, kt + 2);
  TWAIT_VM(0);   // no staging in flight when the workgroup ends

  const float cnt = (float)a.count;
  const bool scaled = a.gmode == 3;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const int rl = rw0 + 32 * (e / 16) + 8 * ((e % 16) / 4) + (e % 4);
    if (rl >= a.R_s || cw >= a.C) continue;
    const float g = gv[e];
    float geff = g;
    if constexpr (SURR) {
      const float dw = wv[e] - a.anchor[(rbase + rl) * a.lda + cw];
      const float bd = a.beta[rbase + rl] * dw;
      geff = g + bd;
    }
    const float cg = cnt * geff;
    const float gupd = cg - w.accD[e];
    const float tot = w.accE[e] + gupd;
    a.Wp[(rbase + rl) * a.ldw + cw] = wv[e] - (scaled ? a.sos * tot : tot);
    a.GH[(rbase + rl) * a.ldgh + cw] = g - w.accZ[e];
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
                                  const float* err, const int* z_nonzero, int z_zero, int gmode,
                                  const float* anchor, int64_t ld_anchor, const float* beta,
                                  double second_order_scale, void* stream) {
  if (!Wp || !GH || !Z || !Hinv_all || !err || !z_nonzero) return RQ_EINVAL;
  if (gmode < 0 || gmode > 3) return RQ_EINVAL;
  if ((gmode == 1 || gmode == 2) && (!anchor || !beta || ld_anchor < C)) return RQ_EINVAL;
  if (R <= 0 || R_s <= 0 || R % R_s != 0 || C <= 0 || ldw < C || ldgh < C) return RQ_EINVAL;
  if (count <= 0 || i1 < 0 || i1 + count > C) return RQ_EINVAL;
  const int i2 = i1 + count;
  if (i2 >= C) return RQ_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (z_zero && (gmode == RQ_GMODE_FROZEN || gmode == RQ_GMODE_BLOCK_GD) && count % 8 == 0 &&
      C % 4 == 0 && i2 % 4 == 0 && al16(Hinv_all) && al16(err)) {
    // Z (and with it GH) identically zero: only W -= f * err Hinv[i1:i2, i2:] remains
    TwArgs w{Wp, ldw, Hinv_all, C, R_s, i1, count, err,
             gmode == RQ_GMODE_BLOCK_GD ? (float)second_order_scale : 1.0f,
             (R_s + TT - 1) / TT, (C - i2 + TT - 1) / TT, 0, i2};
    w.total = w.nrt * w.nct * (R / R_s);
    hipLaunchKernelGGL(k_trailing_w, dim3(w.total), dim3(256), 0, s, w);
    RQ_CHECK_LAUNCH();
    return RQ_OK;
  }
  if (count % 8 == 0 && C % 4 == 0 && i1 % 4 == 0 && ldgh % 4 == 0 && al16(Hinv_all) && al16(err) &&
      al16(Z)) {
    // the GPTQ+ terms present (or not known to be zero): three k-ordered chains per output
    TzArgs z{Wp, ldw, GH, Z, ldgh, Hinv_all, C, R_s, i1, count, err, gmode, anchor, ld_anchor, beta,
             (float)second_order_scale, (R_s + TZR - 1) / TZR, (C - i2 + TZC - 1) / TZC, 0};
    z.total = z.nrt * z.nct * (R / R_s);
    if (gmode == RQ_GMODE_SURROGATE_BLOCK || gmode == RQ_GMODE_SURROGATE_ONLINE)
      hipLaunchKernelGGL(k_trailing_z<true>, dim3(z.total), dim3(256), 0, s, z);
    else
      hipLaunchKernelGGL(k_trailing_z<false>, dim3(z.total), dim3(256), 0, s, z);
    RQ_CHECK_LAUNCH();
    return RQ_OK;
  }
  TrArgs a{Wp, ldw, GH, Z, ldgh, Hinv_all, C, R, R_s, i1, count, err, z_nonzero, gmode,
           anchor, ld_anchor, beta, (float)second_order_scale};
  dim3 grid((C - i2 + 63) / 64, (R_s + 63) / 64, R / R_s), block(256);
  hipLaunchKernelGGL(k_trailing, grid, block, 0, s, a);
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}

extern "C" int rq_quant_block_lookahead(float* Wp, int64_t ldw, const float* Hinv_all, int C, int R, int R_s,
                                        int i1, int count, const float* err, int count_next, int qmode,
                                        const float* scale, const int32_t* col_group, float* dyn_scale,
                                        int maxq, int sym, int atomic, int16_t* codes, float* err_next,
                                        void* stream) {
  if (!Wp || !Hinv_all || !err || !codes || !err_next || err == err_next) return RQ_EINVAL;
  if (R <= 0 || R_s <= 0 || R % R_s != 0 || C <= 0 || ldw < C) return RQ_EINVAL;
  if (count <= 0 || count > QB_MAXB || i1 < 0 || count_next <= 0 || count_next > QB_MAXB) return RQ_EINVAL;
  const int i1n = i1 + count, cbeg = i1n + count_next;
  if (cbeg > C || maxq <= 0 || qmode < 0 || qmode > 2) return RQ_EINVAL;
  if (qmode == RQ_QMODE_CHANNEL && !scale) return RQ_EINVAL;
  if (qmode == RQ_QMODE_STATIC && (!scale || !col_group)) return RQ_EINVAL;
  if (qmode == RQ_QMODE_DYNAMIC && !dyn_scale) return RQ_EINVAL;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  // the wide part runs k_trailing_w's tiles: its shape conditions
  if (count % 8 || C % 4 || cbeg % 4 || !al16(Hinv_all) || !al16(err)) return RQ_EINVAL;
  QBArgs q{};
  q.Wp = Wp;
  q.ldw = ldw;
  q.Hinv = Hinv_all;
  q.C = C;
  q.GH = nullptr;
  q.Z = nullptr;
  q.ldgh = C;
  q.R = R;
  q.R_s = R_s;
  q.i1 = i1n;
  q.count = count_next;
  q.qmode = qmode;
  q.scale = scale;
  q.col_group = col_group;
  q.dyn_scale = dyn_scale;
  q.maxq = (float)maxq;
  q.sym = sym;
  q.atomic = atomic;
  q.z_nonzero = nullptr;
  q.codes = codes;
  q.err = err_next;
  q.anchor = nullptr;
  q.lda = C;
  q.beta = nullptr;
  q.sos = 1.0f;
  q.near_err = err;
  q.near_i1 = i1;
  q.near_count = count;
  q.zero_terms = 1;
  TwArgs w{Wp, ldw, Hinv_all, C, R_s, i1, count, err, 1.0f, (R_s + TT - 1) / TT, (C - cbeg + TT - 1) / TT, 0,
           cbeg};
  w.total = (cbeg < C) ? w.nrt * w.nct * (R / R_s) : 0;
  const int nqx = (R_s + 256 / QL - 1) / (256 / QL), nq = nqx * (R / R_s);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (count_next <= 2 * QL)
    hipLaunchKernelGGL(k_block_lookahead<2>, dim3(nq + w.total), dim3(256), 0, s, q, w, nqx, nq);
  else
    hipLaunchKernelGGL(k_block_lookahead<8>, dim3(nq + w.total), dim3(256), 0, s, q, w, nqx, nq);
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}
