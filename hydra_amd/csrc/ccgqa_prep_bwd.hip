// Backward of the CCGQA q/k/v preparation (hydra_ccgqa_prep_fwd) on gfx950,
// i.e. what torch autograd computes through CCGQAAttention.forward between
// the qkv GEMM and the attention core (reference:
// hydra/attention/backends/ccgqa/attention.py:205-266 and
// kernels/fused_conv.py:39-62, trained through autograd there).
//
// Split in three kinds of work:
//   * hydra_ccgqa_prep_bwd: the pointwise chain, one token per wave --
//     RoPE transpose, F.normalize backward (with the temperature and its
//     gradient), QK-mean backward, value-shift backward.  It reads the conv
//     outputs (recomputed by the caller with the forward kernel) and the
//     pre-conv q0/k0 from qkv, and writes the gradient of the conv outputs,
//     the QK-mean and v parts of grad(qkv) and a per-token partial of
//     grad(temperature).
//   * hydra_causal_im2col / hydra_causal_col2im: the k-tap causal conv as a
//     GEMM over [tap, channel] columns (per group), so the conv backward is
//     plain library GEMMs: dX = col2im(dY W), dW = dY^T im2col(X).
//   * the GEMMs themselves (hipBLASLt through the caller).
#include "common.h"

#include <algorithm>

namespace hydra {

constexpr int kPbThreads = 256;  // 4 waves, one token per wave at a time

template <typename T>
__device__ __forceinline__ float rd(float v) {
  return to_f32(from_f32<T>(v));
}

// Orders one wave's LDS writes before its later LDS reads by other lanes
// (a wave-scope fence plus a compiler scheduling barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// One token (b, s) per wave.  LDS per wave: xs[CW] (the pre-norm value
// qc/kc), gs[CW] (incoming gradient after the RoPE transpose, then the
// gradient of qc/kc), hs[2*NH] (per-head norm and projection).
template <typename T>
__global__ __launch_bounds__(kPbThreads) void ccgqa_prep_bwd_kernel(
    const T* __restrict__ qkv, int64_t qkv_rs, const T* __restrict__ y2q,
    const T* __restrict__ y2k, const T* __restrict__ temp, const float* __restrict__ cs,
    const float* __restrict__ sn, int64_t cs_rs, const T* __restrict__ dq,
    const T* __restrict__ dk, const T* __restrict__ dv, T* __restrict__ dy,
    T* __restrict__ dqkv, int64_t dqkv_rs, float* __restrict__ dtemp_tok, int B, int S, int Hq,
    int Hkv, int hd, int flags) {
  extern __shared__ float pb_smem[];
  const int L = Hq * hd, K = Hkv * hd, CW = L + K, NH = Hq + Hkv;
  const int G = Hq / Hkv;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float* xs = pb_smem + wave * (2 * CW + 2 * NH);
  float* gs = xs + CW;
  float* hs = gs + CW;  // [NH] 1/n (0: below eps), [NH] projection
  const bool convs = flags & HYDRA_CCGQA_CONVS;
  const bool qk_mean = flags & HYDRA_CCGQA_QK_MEAN;
  const bool vshift = flags & HYDRA_CCGQA_VALUE_SHIFT;
  const bool qk_norm = flags & HYDRA_CCGQA_QK_NORM;
  const bool rope = flags & HYDRA_CCGQA_ROPE;
  const float tval = (qk_norm && temp) ? to_f32(temp[0]) : 1.f;
  const float inv_q = 1.f / static_cast<float>(Hq), inv_k = 1.f / static_cast<float>(Hkv);
  const int64_t ntok = static_cast<int64_t>(B) * S;
  for (int64_t tok = static_cast<int64_t>(blockIdx.x) * (kPbThreads / 64) + wave; tok < ntok;
       tok += static_cast<int64_t>(gridDim.x) * (kPbThreads / 64)) {
    const int b = static_cast<int>(tok / S), s = static_cast<int>(tok - static_cast<int64_t>(b) * S);
    const T* xr = qkv + tok * qkv_rs;
    // ---- A: pre-norm value (conv output + QK-mean term) and the gradient
    // after the RoPE transpose, a channel pair per lane
    for (int p = lane; p < CW / 2; p += 64) {
      const int ch = 2 * p;
      const bool is_k = ch >= L;
      const int h = (is_k ? ch - L : ch) / hd, d = (is_k ? ch - L : ch) - h * hd;
      float x0, x1;
      if (convs) {
        const T* y = is_k ? y2k + ((static_cast<int64_t>(b) * Hkv + h) * S + s) * hd + d
                          : y2q + ((static_cast<int64_t>(b) * Hq + h) * S + s) * hd + d;
        x0 = to_f32(y[0]);
        x1 = to_f32(y[1]);
      } else {
        x0 = to_f32(xr[ch]);
        x1 = to_f32(xr[ch + 1]);
      }
      if (qk_mean) {
        float t0, t1;
        if (G == 1) {  // (q0_h + k0_h) / 2 for q and k head h
          t0 = rd<T>(0.5f * rd<T>(to_f32(xr[h * hd + d]) + to_f32(xr[L + h * hd + d])));
          t1 = rd<T>(0.5f * rd<T>(to_f32(xr[h * hd + d + 1]) + to_f32(xr[L + h * hd + d + 1])));
        } else {  // q heads: mean of the k heads; k heads: mean of the q heads
          const int nh = is_k ? Hq : Hkv;
          const T* src = xr + (is_k ? 0 : L) + d;
          float a0 = 0.f, a1 = 0.f;
          for (int hx = 0; hx < nh; ++hx) {
            a0 += to_f32(src[hx * hd]);
            a1 += to_f32(src[hx * hd + 1]);
          }
          const float inv = is_k ? inv_q : inv_k;
          t0 = rd<T>(0.5f * rd<T>(a0 * inv));
          t1 = rd<T>(0.5f * rd<T>(a1 * inv));
        }
        x0 = rd<T>(x0 + t0);
        x1 = rd<T>(x1 + t1);
      }
      const T* gsrc = is_k ? dk + ((static_cast<int64_t>(b) * Hkv + h) * S + s) * hd + d
                           : dq + ((static_cast<int64_t>(b) * Hq + h) * S + s) * hd + d;
      float g0 = to_f32(gsrc[0]), g1 = to_f32(gsrc[1]);
      if (rope) {  // forward (x0,x1) -> (x0 c - x1 s, x0 s + x1 c); its transpose
        const float c = cs[static_cast<int64_t>(s) * cs_rs + d / 2];
        const float sv = sn[static_cast<int64_t>(s) * cs_rs + d / 2];
        const float r0 = g0 * c + g1 * sv, r1 = g1 * c - g0 * sv;
        g0 = r0;
        g1 = r1;
      }
      xs[ch] = x0;
      xs[ch + 1] = x1;
      gs[ch] = g0;
      gs[ch + 1] = g1;
    }
    wave_sync();
    // ---- B: per head, F.normalize backward terms (a head per lane)
    if (qk_norm) {
      float dtemp = 0.f;
      for (int hh = lane; hh < NH; hh += 64) {
        const bool is_k = hh >= Hq;
        const float* x = xs + hh * hd;
        const float* g = gs + hh * hd;
        float ss = 0.f;
        for (int d = 0; d < hd; ++d) ss = fmaf(x[d], x[d], ss);
        const float n = __builtin_sqrtf(ss);
        // forward: x / max(n, 1e-12) (the norm rounded to the working dtype)
        const float den = fmaxf(rd<T>(n), 1e-12f);
        float dot = 0.f, dt = 0.f;
        for (int d = 0; d < hd; ++d) {
          const float xh = x[d] / den;
          dot = fmaf(xh, g[d], dot);
          if (is_k) dt = fmaf(rd<T>(xh), g[d], dt);  // k = rd(x/den) * temperature
        }
        if (is_k) {
          dtemp += dt;
          dot *= tval;
        }
        // below eps the divisor is the constant eps: no projection term
        hs[hh] = 1.f / den;
        hs[NH + hh] = rd<T>(n) > 1e-12f ? dot : 0.f;
      }
      // the sum over the token's k heads: lanes < NH hold the parts
      for (int off = 32; off > 0; off >>= 1) dtemp += __shfl_xor(dtemp, off);
      if (lane == 0 && dtemp_tok) dtemp_tok[tok] = dtemp;
    }
    wave_sync();
    // ---- C: gradient of the pre-norm value; gradient of the conv output
    for (int p = lane; p < CW / 2; p += 64) {
      const int ch = 2 * p;
      const int hh = ch / hd;  // q heads then k heads
      float g0 = gs[ch], g1 = gs[ch + 1];
      if (qk_norm) {
        const bool is_k = hh >= Hq;
        const float rinv = hs[hh], dot = hs[NH + hh];
        const float sc = is_k ? tval : 1.f;
        g0 = (g0 * sc - xs[ch] * rinv * dot) * rinv;
        g1 = (g1 * sc - xs[ch + 1] * rinv * dot) * rinv;
      }
      gs[ch] = g0;
      gs[ch + 1] = g1;
      if (convs) {
        T* o = dy + tok * CW + ch;
        o[0] = from_f32<T>(g0);
        o[1] = from_f32<T>(g1);
      }
    }
    wave_sync();
    // ---- D: q0/k0 parts of grad(qkv): QK-mean (+ the direct path without convs)
    T* gr = dqkv + tok * dqkv_rs;
    for (int p = lane; p < CW / 2; p += 64) {
      const int ch = 2 * p;
      const bool is_k = ch >= L;
      const int h = (is_k ? ch - L : ch) / hd, d = (is_k ? ch - L : ch) - h * hd;
      float m0 = 0.f, m1 = 0.f;
      if (qk_mean) {
        if (G == 1) {  // m = (q0 + k0)/2 feeds q and k of head h
          m0 = 0.5f * (gs[h * hd + d] + gs[L + h * hd + d]);
          m1 = 0.5f * (gs[h * hd + d + 1] + gs[L + h * hd + d + 1]);
        } else {
          // q0 channel: through the q mean into every k head; k0 channel:
          // through the k mean into every q head
          const int nh = is_k ? Hq : Hkv;
          const float* src = gs + (is_k ? 0 : L) + d;
          for (int hx = 0; hx < nh; ++hx) {
            m0 += src[hx * hd];
            m1 += src[hx * hd + 1];
          }
          const float inv = is_k ? inv_k : inv_q;
          m0 *= 0.5f * inv;
          m1 *= 0.5f * inv;
        }
      }
      if (!convs) {
        m0 += gs[ch];
        m1 += gs[ch + 1];
      }
      gr[ch] = from_f32<T>(m0);
      gr[ch + 1] = from_f32<T>(m1);
    }
    // ---- E: v part (value shift: the second half came from token s - 1)
    for (int c = lane; c < K; c += 64) {
      const int j = c / hd, d = c - j * hd;
      float g = 0.f;
      if (vshift && c >= K / 2) {
        if (s + 1 < S) g = to_f32(dv[((static_cast<int64_t>(b) * Hkv + j) * S + s + 1) * hd + d]);
      } else {
        g = to_f32(dv[((static_cast<int64_t>(b) * Hkv + j) * S + s) * hd + d]);
      }
      gr[CW + c] = from_f32<T>(g);
    }
    wave_sync();  // the next token rewrites xs/gs
  }
}

// out[g][n][t*cg + c] = x[b, s + t - 2, g*cg + c] (0 before the row start),
// n = b*S + s.
template <typename T>
__global__ __launch_bounds__(256) void causal_im2col_kernel(const T* __restrict__ x, int64_t x_rs,
                                                           T* __restrict__ out, int64_t N, int S,
                                                           int G, int cg, int taps, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int w = taps * cg;
  const int64_t gn = i / w;
  const int col = static_cast<int>(i - gn * w);
  const int g = static_cast<int>(gn / N);
  const int64_t n = gn - static_cast<int64_t>(g) * N;
  const int t = col / cg, c = col - t * cg;
  const int s = static_cast<int>(n % S);
  const int back = taps - 1 - t;  // tap t reads the token taps-1-t back
  out[i] = s >= back ? x[(n - back) * x_rs + g * cg + c] : from_f32<T>(0.f);
}

// out[b, s, g*cg + c] (+)= sum_t in[g][b*S + s + taps-1-t][t*cg + c] over
// the taps whose output token s + taps-1-t lies in the row.
template <typename T>
__global__ __launch_bounds__(256) void causal_col2im_kernel(const T* __restrict__ in,
                                                           T* __restrict__ out, int64_t out_rs,
                                                           int64_t N, int S, int G, int cg, int taps,
                                                           int accumulate, int64_t total) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int C = G * cg;
  const int64_t n = i / C;
  const int ch = static_cast<int>(i - n * C);
  const int g = ch / cg, c = ch - g * cg;
  const int s = static_cast<int>(n % S);
  const int w = taps * cg;
  const T* base = in + static_cast<int64_t>(g) * N * w;
  float acc = 0.f;
  for (int t = 0; t < taps; ++t) {
    const int fwd = taps - 1 - t;  // output token s + fwd read this input at tap t
    if (s + fwd < S) acc += to_f32(base[(n + fwd) * w + t * cg + c]);
  }
  T* o = out + n * out_rs + ch;
  if (accumulate) acc += to_f32(*o);
  *o = from_f32<T>(acc);
}

}  // namespace hydra

using namespace hydra;

extern "C" int hydra_ccgqa_prep_bwd(const void* qkv, int64_t qkv_rs, const void* y2q,
                                    const void* y2k, const void* temp, const float* cos,
                                    const float* sin, int64_t cs_rs, const void* dq,
                                    const void* dk, const void* dv, void* dy, void* dqkv,
                                    int64_t dqkv_rs, float* dtemp_tok, int64_t B, int64_t S,
                                    int64_t Hq, int64_t Hkv, int64_t hd, int flags, int dtype,
                                    void* stream) {
  HYDRA_REQUIRE(B >= 0 && S >= 0 && Hq >= 1 && Hkv >= 1 && hd >= 2 && hd % 2 == 0,
                "ccgqa_prep_bwd: bad size");
  HYDRA_REQUIRE(Hq % Hkv == 0, "ccgqa_prep_bwd: n_heads must be a multiple of n_kv_heads");
  HYDRA_REQUIRE((flags & ~127) == 0, "ccgqa_prep_bwd: unknown flag bits");
  HYDRA_REQUIRE(!(flags & HYDRA_CCGQA_V_TRANSPOSED), "ccgqa_prep_bwd: dv must be [B, Hkv, S, hd]");
  const int64_t L = Hq * hd, K = Hkv * hd, CW = L + K;
  HYDRA_REQUIRE(CW <= 4096, "ccgqa_prep_bwd: q + k channels must be <= 4096");
  HYDRA_REQUIRE(qkv_rs >= CW + K && dqkv_rs >= CW + K, "ccgqa_prep_bwd: row stride smaller than L + 2K");
  if (B * S == 0) return HYDRA_OK;
  HYDRA_REQUIRE(qkv && dq && dk && dv && dqkv, "ccgqa_prep_bwd: null pointer");
  HYDRA_REQUIRE(!(flags & HYDRA_CCGQA_CONVS) || (y2q && y2k && dy), "ccgqa_prep_bwd: conv outputs required");
  HYDRA_REQUIRE(!(flags & HYDRA_CCGQA_QK_NORM) || temp, "ccgqa_prep_bwd: temperature required");
  HYDRA_REQUIRE(!(flags & HYDRA_CCGQA_ROPE) || (cos && sin && cs_rs >= hd / 2),
                "ccgqa_prep_bwd: cos/sin [S, hd/2] required");
  HYDRA_REQUIRE(B * S < (int64_t(1) << 31), "ccgqa_prep_bwd: too many tokens");
  auto st = static_cast<hipStream_t>(stream);
  const size_t lds = static_cast<size_t>(kPbThreads / 64) * (2 * CW + 2 * (Hq + Hkv)) * sizeof(float);
  const int64_t ntok = B * S;
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>((ntok + 3) / 4, 8192));
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    auto kern = ccgqa_prep_bwd_kernel<T>;
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)) != hipSuccess)
      return fail(HYDRA_ERR_LAUNCH, "ccgqa_prep_bwd: cannot set the kernel's LDS size");
    kern<<<grid, kPbThreads, lds, st>>>(
        static_cast<const T*>(qkv), qkv_rs, static_cast<const T*>(y2q), static_cast<const T*>(y2k),
        static_cast<const T*>(temp), cos, sin, cs_rs, static_cast<const T*>(dq),
        static_cast<const T*>(dk), static_cast<const T*>(dv), static_cast<T*>(dy),
        static_cast<T*>(dqkv), dqkv_rs, dtemp_tok, (int)B, (int)S, (int)Hq, (int)Hkv, (int)hd, flags);
    return check_launch("ccgqa_prep_bwd_kernel");
  });
}

extern "C" int hydra_causal_im2col(const void* x, int64_t x_rs, void* out, int64_t B, int64_t S,
                                   int64_t G, int64_t cg, int64_t taps, int dtype, void* stream) {
  HYDRA_REQUIRE(B >= 0 && S >= 0 && G >= 1 && cg >= 1, "causal_im2col: bad size");
  HYDRA_REQUIRE(taps >= 1 && taps <= 16, "causal_im2col: taps must be in [1, 16]");
  HYDRA_REQUIRE(x_rs >= G * cg, "causal_im2col: row stride smaller than G * cg");
  const int64_t total = G * B * S * taps * cg;
  if (total == 0) return HYDRA_OK;
  HYDRA_REQUIRE(x && out, "causal_im2col: null pointer");
  HYDRA_REQUIRE(S < (int64_t(1) << 31) && G * cg < (int64_t(1) << 31), "causal_im2col: too large");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    causal_im2col_kernel<T><<<static_cast<unsigned>((total + 255) / 256), 256, 0, st>>>(
        static_cast<const T*>(x), x_rs, static_cast<T*>(out), B * S, (int)S, (int)G, (int)cg, (int)taps,
        total);
    return check_launch("causal_im2col_kernel");
  });
}

extern "C" int hydra_causal_col2im(const void* in, void* out, int64_t out_rs, int64_t B, int64_t S,
                                   int64_t G, int64_t cg, int64_t taps, int accumulate, int dtype,
                                   void* stream) {
  HYDRA_REQUIRE(B >= 0 && S >= 0 && G >= 1 && cg >= 1, "causal_col2im: bad size");
  HYDRA_REQUIRE(taps >= 1 && taps <= 16, "causal_col2im: taps must be in [1, 16]");
  HYDRA_REQUIRE(out_rs >= G * cg, "causal_col2im: row stride smaller than G * cg");
  const int64_t total = B * S * G * cg;
  if (total == 0) return HYDRA_OK;
  HYDRA_REQUIRE(in && out, "causal_col2im: null pointer");
  HYDRA_REQUIRE(S < (int64_t(1) << 31) && G * cg < (int64_t(1) << 31), "causal_col2im: too large");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    causal_col2im_kernel<T><<<static_cast<unsigned>((total + 255) / 256), 256, 0, st>>>(
        static_cast<const T*>(in), static_cast<T*>(out), out_rs, B * S, (int)S, (int)G, (int)cg,
        (int)taps, accumulate, total);
    return check_launch("causal_col2im_kernel");
  });
}
