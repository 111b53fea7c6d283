// The pieces of the gradient-refresh g_update modes that run between the caller's layer
// backward calls (gptq_utils/gptq_plus_utils.py:1389-1448 block_backward, :1572-1848
// block_gd):
//
// k_current_weight  the "current effective weight" the refresh sees: quantized columns
//                   (permuted index j < i_q) replaced by Q = fl(scale * code), the rest the
//                   live working weight, optionally un-permuted (the snapshot handed to the
//                   caller) and optionally minus a reference weight (the hessian
//                   regularizer's W - W_fp).  One pass, HBM-bound.
// k_gather_cols     dst[r, j] = src[r, perm[j]]: the refreshed gradient in act_order's order.
// k_kfac_curvature  H-Adam's curvature row, diag(H_sub) normalised to unit mean + damping
//                   (:4601-4640, input factor only as called at :1148), one workgroup per
//                   subgroup.
// k_block_gd_step   the optimizer step and first-order regularizer on the trailing columns
//                   [i2, C) of every row, fused into one elementwise pass (:616-655, :730-796,
//                   :1828-1834): clip, SGD / Adam / H-Adam moments, l2 / hessian /
//                   quant-error gate (+ sine) terms, W -= update.  HBM-bound.
// The hessian regularizer's (W - W_fp) H_reg[:, i2:] product is an fp32 MFMA GEMM
// (gemm_tile.h), batched over subgroups.
//
// Scalars follow torch's promotion of Python floats: every scalar operand is first rounded
// to fp32, and each tensor op rounds once (Tensor.add_(x, alpha=a) is a fused multiply-add
// in torch's vectorised CPU kernels, addcmul_ is not).
#include "gemm_tile.h"

namespace {

__device__ __forceinline__ float qscale_at(int qmode, const float* scale, const int32_t* col_group,
                                           const float* dyn_scale, int bs, int R, int r, int64_t j) {
  if (qmode == RQ_QMODE_CHANNEL) return scale[r];
  if (qmode == RQ_QMODE_STATIC) return scale[(int64_t)col_group[j] * R + r];
  return dyn_scale[(j / bs) * (int64_t)R + r];
}

__global__ __launch_bounds__(256) void k_current_weight(
    const float* __restrict__ Wp, int64_t ldw, const int16_t* __restrict__ codes, int R, int C,
    int i_q, int qmode, const float* __restrict__ scale, const int32_t* __restrict__ col_group,
    const float* __restrict__ dyn_scale, int bs, const int64_t* __restrict__ invperm,
    const float* __restrict__ sub_ref, int64_t ld_ref, float* __restrict__ out, int64_t ldo) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  const int64_t j = invperm ? invperm[c] : c;
  for (int r = blockIdx.y; r < R; r += gridDim.y) {
    float v;
    if (j < i_q) {
      const int16_t ci = codes[(int64_t)r * C + j];
      const float code = (ci == RQ_CODE_NAN) ? __builtin_nanf("") : (float)ci;
      v = qscale_at(qmode, scale, col_group, dyn_scale, bs, R, r, j) * code;
    } else {
      v = Wp[(int64_t)r * ldw + j];
    }
    if (sub_ref) v = v - sub_ref[(int64_t)r * ld_ref + c];
    out[(int64_t)r * ldo + c] = v;
  }
}

__global__ __launch_bounds__(256) void k_gather_cols(const float* __restrict__ src, int64_t lds,
                                                     const int64_t* __restrict__ perm, int R, int C,
                                                     float* __restrict__ dst, int64_t ldd) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= C) return;
  const int64_t c = perm ? perm[j] : j;
  for (int r = blockIdx.y; r < R; r += gridDim.y) dst[(int64_t)r * ldd + j] = src[(int64_t)r * lds + c];
}

// curvature[s][j] = clamp_min(d_j, 0) / max(mean(clamp_min(d, 0)), 1e-12) + damping,
// d = the diagonal of H_work[s] (dead-column fixed and permuted, before any damping)
__global__ __launch_bounds__(256) void k_kfac_curvature(const float* __restrict__ H, int C,
                                                        float damping, float* __restrict__ curv) {
  __shared__ double part[256];
  const int s = blockIdx.x;
  const float* Hs = H + (int64_t)s * C * C;
  double acc = 0.0;
  for (int j = threadIdx.x; j < C; j += 256) acc += (double)fmaxf(Hs[(int64_t)j * C + j], 0.0f);
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  const float mean = fmaxf((float)(part[0] / (double)C), 1e-12f);
  for (int j = threadIdx.x; j < C; j += 256) {
    float a = fmaxf(Hs[(int64_t)j * C + j], 0.0f) / mean;
    if (damping > 0.0f) a = a + damping;
    curv[(int64_t)s * C + j] = a;
  }
}

struct GdArgs {
  float* Wp;
  int64_t ldw;
  int R, R_s, C, i2;
  const float* grad;   // refreshed gradient, natural column order [R, C]
  int64_t ldg;
  const int64_t* perm; // act_order permutation (NULL = identity)
  int opt;             // 0 sgd, 1 adam, 2 h_adam
  float lr, clip, b1, one_m_b1, b2, one_m_b2, eps, step_size, sqrt_bc2;
  float* exp_avg;      // [R, C] permuted
  float* exp_avg_sq;   // [R, C] permuted (adam)
  const float* curv;   // [G, C] (h_adam)
  int reg;             // 0 none, 1 l2, 2 hessian, 3 gate, 4 gate + sine
  float lr_lam;        // fl32(lr * lambda)
  const float* w_fp;   // [R, C] permuted (l2)
  int64_t ld_fp;
  const float* hreg;   // [R, C - i2] = (W - W_fp) H_reg[:, i2:] (hessian)
  int64_t ld_hreg;
  // gate maps: qmode channel -> gscale[r] / gzero[r]; static -> gscale[col_group[j] * R + r]
  int gqmode;
  const float* gscale;
  const float* gzero;
  const int32_t* col_group;
  float maxq;
  int sym;
  float floor_, one_m_floor, neg_sharp, amp, two_pi;
  // optional statistics planes [4][R][C - i2]: the optimizer step (after clipping), the applied
  // update, the regularizer part (l2 / hessian term or gated - step) and the sine part
  float* parts;
};

__global__ __launch_bounds__(256) void k_block_gd_step(GdArgs a) {
  const int jj = blockIdx.x * 256 + threadIdx.x;
  const int j = a.i2 + jj;
  if (j >= a.C) return;
  const int64_t gc = a.perm ? a.perm[j] : j;
  for (int r = blockIdx.y; r < a.R; r += gridDim.y) {
    const int64_t o = (int64_t)r * a.C + j;
    const int64_t ow = (int64_t)r * a.ldw + j;
    float g = a.grad[(int64_t)r * a.ldg + gc];
    if (a.clip > 0.0f && g == g) g = fminf(fmaxf(g, -a.clip), a.clip);   // clamp; NaN stays NaN
    float upd;
    if (a.opt == 0) {
      upd = a.lr * g;
    } else {
      float m = a.exp_avg[o] * a.b1;
      m = __builtin_fmaf(g, a.one_m_b1, m);                 // add_(g, alpha=1 - b1)
      a.exp_avg[o] = m;
      float denom;
      if (a.opt == 2) {
        denom = __builtin_sqrtf(a.curv[(int64_t)(r / a.R_s) * a.C + j]) + a.eps;
      } else {
        float v = a.exp_avg_sq[o] * a.b2;
        v = v + (a.one_m_b2 * g) * g;                        // addcmul_(g, g, value=1 - b2)
        a.exp_avg_sq[o] = v;
        denom = __builtin_sqrtf(v) / a.sqrt_bc2;
        denom = denom + a.eps;
      }
      upd = a.step_size * (m / denom);
    }
    const float raw = upd;
    float reg_part = 0.0f, sine_part = 0.0f;
    const float w = a.Wp[ow];
    if (a.reg == 1) {
      reg_part = a.lr_lam * (w - a.w_fp[(int64_t)r * a.ld_fp + j]);
      upd = upd + reg_part;
    } else if (a.reg == 2) {
      reg_part = a.lr_lam * a.hreg[(int64_t)r * a.ld_hreg + jj];
      upd = upd + reg_part;
    } else if (a.reg >= 3) {
      float s, z;
      if (a.gqmode == RQ_QMODE_CHANNEL) {
        s = a.gscale[r];
        z = a.gzero[r];
      } else {
        const int64_t gi = (int64_t)a.col_group[j] * a.R + r;
        s = a.gscale[gi];
        z = a.gzero[gi];
      }
      const float sc = (s == s) ? fmaxf(s, 1e-8f) : s;      // clamp(min=1e-8); NaN stays NaN
      float qn;
      if (a.sym) {
        qn = sc * fminf(fmaxf(__builtin_rintf(w / sc), -(a.maxq + 1.0f)), a.maxq);
      } else {
        const float qi = fminf(fmaxf(__builtin_rintf(w / sc) + z, 0.0f), a.maxq);
        qn = sc * (qi - z);
      }
      const float dist = fabsf(w - qn) / sc;
      const float gate = a.floor_ + a.one_m_floor * (1.0f - expf(a.neg_sharp * dist));
      const float gated = upd * gate;
      reg_part = gated - upd;
      if (a.reg == 4) {
        const float ws = w / sc;
        const float phase = a.sym ? a.two_pi * ws : a.two_pi * (ws + z);
        const float sine = (a.amp * (a.two_pi / sc)) * sinf(phase);
        sine_part = a.lr * sine;
        upd = gated + sine_part;
      } else {
        upd = gated;
      }
    }
    a.Wp[ow] = w - upd;
    if (a.parts) {
      const int64_t n = (int64_t)a.R * (a.C - a.i2), e = (int64_t)r * (a.C - a.i2) + jj;
      a.parts[e] = raw;
      a.parts[n + e] = upd;
      a.parts[2 * n + e] = reg_part;
      a.parts[3 * n + e] = sine_part;
    }
  }
}

inline int rows_grid(int rows) { return rows < 1024 ? rows : 1024; }

}  // namespace

extern "C" int rq_current_weight(const float* Wp, int64_t ldw, const int16_t* codes, int R, int C,
                                 int i_q, int qmode, const float* scale, const int32_t* col_group,
                                 const float* dyn_scale, int blocksize, const int64_t* invperm,
                                 const float* sub_ref, int64_t ld_ref, float* out, int64_t ldo,
                                 void* stream) {
  if (!Wp || !codes || !out || R <= 0 || C <= 0 || ldw < C || ldo < C) return RQ_EINVAL;
  if (i_q < 0 || i_q > C || qmode < 0 || qmode > 2) return RQ_EINVAL;
  if (i_q > 0) {
    if (qmode == RQ_QMODE_CHANNEL && !scale) return RQ_EINVAL;
    if (qmode == RQ_QMODE_STATIC && (!scale || !col_group)) return RQ_EINVAL;
    if (qmode == RQ_QMODE_DYNAMIC && (!dyn_scale || blocksize <= 0)) return RQ_EINVAL;
  }
  if (sub_ref && ld_ref < C) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((C + 255) / 256, rows_grid(R)), block(256);
  hipLaunchKernelGGL(k_current_weight, grid, block, 0, s, Wp, ldw, codes, R, C, i_q, qmode, scale,
                     col_group, dyn_scale, blocksize, invperm, sub_ref, ld_ref, out, ldo);
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}

extern "C" int rq_gather_cols(const float* src, int64_t lds, const int64_t* perm, int R, int C,
                              float* dst, int64_t ldd, void* stream) {
  if (!src || !dst || R <= 0 || C <= 0 || lds < C || ldd < C) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((C + 255) / 256, rows_grid(R)), block(256);
  hipLaunchKernelGGL(k_gather_cols, grid, block, 0, s, src, lds, perm, R, C, dst, ldd);
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}

extern "C" int rq_kfac_curvature(const float* H_work, int C, int nsub, double damping, float* curv,
                                 void* stream) {
  if (!H_work || !curv || C <= 0 || nsub <= 0) return RQ_EINVAL;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_kfac_curvature, dim3(nsub), dim3(256), 0, s, H_work, C, (float)damping, curv);
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}

extern "C" int rq_hessian_reg_gemm(const float* diff, int64_t ldd, const float* H_reg, int C, int R,
                                   int R_s, int i2, float* out, int64_t ldo, void* stream) {
  if (!diff || !H_reg || !out || C <= 0 || R <= 0 || R_s <= 0 || R % R_s) return RQ_EINVAL;
  if (ldd < C || i2 < 0 || i2 >= C || ldo < C - i2) return RQ_EINVAL;
  // out[s] = diff[s] (R_s x C) * H_reg[s][:, i2:] (C x (C - i2)), subgroups in grid z
  rq::GemmArgs<float> g = rq::gemm_args<float>(diff, ldd, H_reg + i2, C, out, ldo, R_s, C - i2, C,
                                               1.0f, rq::EPI_STORE);
  g.sA = (int64_t)R_s * ldd;
  g.sB = (int64_t)C * C;
  g.sC = (int64_t)R_s * ldo;
  return rq::launch_gemm(g, false, false, reinterpret_cast<hipStream_t>(stream), R / R_s);
}

extern "C" int rq_block_gd_step(float* Wp, int64_t ldw, int R, int R_s, int C, int i2,
                                const float* grad, int64_t ldg, const int64_t* perm, int optimizer,
                                int step, double lr, double grad_clip, float* exp_avg,
                                float* exp_avg_sq, const float* curvature, int reg_strategy,
                                double reg_lambda, const float* w_fp, int64_t ld_fp,
                                const float* hreg, int64_t ld_hreg, int gate_qmode,
                                const float* gate_scale, const float* gate_zero,
                                const int32_t* col_group, int maxq, int sym, double gate_floor,
                                double gate_sharpness, double sine_amp, float* stats_parts,
                                void* stream) {
  if (!Wp || !grad || R <= 0 || R_s <= 0 || R % R_s || C <= 0 || ldw < C || ldg < C) return RQ_EINVAL;
  if (i2 < 0 || i2 > C || optimizer < 0 || optimizer > 2 || reg_strategy < 0 || reg_strategy > 4)
    return RQ_EINVAL;
  if (i2 == C) return RQ_OK;
  if (optimizer >= 1 && (!exp_avg || step <= 0)) return RQ_EINVAL;
  if (optimizer == 1 && !exp_avg_sq) return RQ_EINVAL;
  if (optimizer == 2 && !curvature) return RQ_EINVAL;
  if (reg_strategy == 1 && (!w_fp || ld_fp < C)) return RQ_EINVAL;
  if (reg_strategy == 2 && (!hreg || ld_hreg < C - i2)) return RQ_EINVAL;
  if (reg_strategy >= 3) {
    if (!gate_scale || !gate_zero) return RQ_EINVAL;
    if (gate_qmode == RQ_QMODE_STATIC && !col_group) return RQ_EINVAL;
    if (gate_qmode != RQ_QMODE_CHANNEL && gate_qmode != RQ_QMODE_STATIC) return RQ_EINVAL;
  }
  const double b1 = 0.9, b2 = 0.999, eps = 1e-8;
  GdArgs a{};
  a.Wp = Wp; a.ldw = ldw; a.R = R; a.R_s = R_s; a.C = C; a.i2 = i2;
  a.grad = grad; a.ldg = ldg; a.perm = perm; a.opt = optimizer;
  a.lr = (float)lr; a.clip = (float)grad_clip; a.b1 = (float)b1; a.one_m_b1 = (float)(1.0 - b1);
  a.b2 = (float)b2; a.one_m_b2 = (float)(1.0 - b2); a.eps = (float)eps;
  if (optimizer >= 1) {
    a.step_size = (float)(lr / (1.0 - pow(b1, step)));     // lr / bias_correction1
    a.sqrt_bc2 = (float)sqrt(1.0 - pow(b2, step));          // math.sqrt(bias_correction2)
  }
  a.exp_avg = exp_avg; a.exp_avg_sq = exp_avg_sq; a.curv = curvature;
  a.reg = reg_strategy; a.lr_lam = (float)(lr * reg_lambda);
  a.w_fp = w_fp; a.ld_fp = ld_fp; a.hreg = hreg; a.ld_hreg = ld_hreg;
  a.gqmode = gate_qmode; a.gscale = gate_scale; a.gzero = gate_zero; a.col_group = col_group;
  a.maxq = (float)maxq; a.sym = sym;
  a.floor_ = (float)gate_floor; a.one_m_floor = (float)(1.0 - gate_floor);
  a.neg_sharp = (float)(-gate_sharpness); a.amp = (float)sine_amp; a.two_pi = (float)(2.0 * M_PI);
  a.parts = stats_parts;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  dim3 grid((C - i2 + 255) / 256, rows_grid(R)), block(256);
  hipLaunchKernelGGL(k_block_gd_step, grid, block, 0, s, a);
  RQ_CHECK_LAUNCH();
  return RQ_OK;
}
