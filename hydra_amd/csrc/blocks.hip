// Row kernels of the HYDRA block compositions on gfx950: the token
// embedding lookup, residual adds fused with the pre-norms (RMSNorm and
// AdaRMSNorm), and the per-token bookkeeping of Mixture-of-Recursions.
//
// References (mcpirate17/HYDRA):
//   _safe_embedding_lookup        hydra/model/framework/model.py:51-73
//   HydraBlock.forward            hydra/model/framework/blocks.py:68-70
//   HydraMoRBlock._forward_mor    hydra/model/framework/blocks.py:614-633
//   RMSNorm / AdaRMSNorm          hydra/layers/common.py:74-118, 121-172
//   MoRRouter.forward             hydra/routing/mixture_of_recursions.py:238-288
//   MoRExecutor.forward           hydra/routing/mixture_of_recursions.py:370-478
//
// Every kernel is HBM-bound: one read of each input row and one write of
// each output row, 16-byte accesses, fp32 arithmetic.  Where the reference
// materialises an intermediate tensor in the model dtype (a residual sum, a
// bf16 AdaRMSNorm step), the value is rounded to that dtype at the same
// point, so the bf16 results follow the reference's rounding sequence.
#include "common.h"

#include <algorithm>

namespace hydra {
namespace {

constexpr int kBlk = 256;

// v rounded to T and back (identity for fp32).
template <typename T>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (sizeof(T) == 4) return v;
  else return to_f32(from_f32<T>(v));
}

// E consecutive elements of W at p (16-byte aligned) as fp32; W is T or
// fp32, so E * sizeof(W) is a multiple of 16.
template <typename W, int E>
__device__ __forceinline__ void load_elems(const W* p, float* out) {
  constexpr int PER = 16 / int(sizeof(W));
  static_assert(E % PER == 0, "load_elems: E must cover whole 16-byte chunks");
#pragma unroll
  for (int i = 0; i < E / PER; ++i) load16<W>(p + i * PER, out + i * PER);
}

enum NormMode { kNormNone = 0, kNormRms = 1, kNormAda = 2 };

// ---------------------------------------------------------------------------
// Embedding: out[r] = table[clamp(ids[r], 0, V-1)] * scale, one rounding
// (model.py:51-73: the ids are always clamped; embedding(x) * scale).
// One thread per 16-byte chunk of an output row.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kBlk) void embed_vec_kernel(
    const int64_t* __restrict__ ids, const T* __restrict__ table, T* __restrict__ out,
    uint32_t total, uint32_t cpr, int64_t vocab, int64_t t_rs, int64_t o_rs, float scale) {
  constexpr int E = Vec<T>::N;
  const uint32_t t = blockIdx.x * kBlk + threadIdx.x;
  if (t >= total) return;
  const uint32_t r = t / cpr, c = t - r * cpr;
  int64_t id = ids[r];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  float f[E];
  load16<T>(table + id * t_rs + c * E, f);
#pragma unroll
  for (int e = 0; e < E; ++e) f[e] *= scale;
  store16<T, true>(out + static_cast<int64_t>(r) * o_rs + c * E, f);
}

template <typename T>
__global__ __launch_bounds__(kBlk) void embed_scalar_kernel(
    const int64_t* __restrict__ ids, const T* __restrict__ table, T* __restrict__ out,
    int64_t total, int64_t dim, int64_t vocab, int64_t t_rs, int64_t o_rs, float scale) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlk + threadIdx.x;
  if (t >= total) return;
  const int64_t r = t / dim, c = t - r * dim;
  int64_t id = ids[r];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  out[r * o_rs + c] = from_f32<T>(to_f32(table[id * t_rs + c]) * scale);
}

// ---------------------------------------------------------------------------
// Residual add + norm.  Per element of a row (each step rounded to T, as the
// reference's tensor ops are):
//   v = x;  v = v + (alpha == 1 ? r : rnd(alpha * r));  v = v + b1;  v = v + b2
// h_out = v (optional); y = norm(v) (optional):
//   RMS: y = v * rsqrt(sum(v^2) / dim + eps) * w, fp32, one rounding
//        (RMSNorm, common.py:74-118, fused_ops.py:969-1007);
//   ADA: AdaRMSNorm._rmsnorm (common.py:153-157) in the input dtype:
//        m = rnd(sum(rnd(v^2)) / dim), s = rnd(rsqrt(rnd(m + eps))),
//        y = rnd(rnd(v * s) * w).
// LPR lanes per row, CPL 16-byte chunks per lane, RI row groups per wave,
// all loads of a wave's row groups issued before its reductions.
// ---------------------------------------------------------------------------
struct ResNormArgs {
  const void* x; int64_t x_rs;
  const void* r; int64_t r_rs; float alpha;
  const void* b1; const void* b2;
  const void* w;
  void* h; int64_t h_rs;
  void* y; int64_t y_rs;
  int64_t rows; int nvec; int dim; float eps;
};

template <typename T, typename WT, int LPR, int CPL, int RI, int NORM>
__global__ __launch_bounds__(kBlk) void resnorm_vec_kernel(ResNormArgs a) {
  constexpr int E = Vec<T>::N;
  constexpr int RPW = 64 / LPR;
  constexpr int RPB = (kBlk / 64) * RPW * RI;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, l = lane % LPR;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * RPB + (wave * RI) * RPW + sub;
  const T* X = static_cast<const T*>(a.x);
  const T* R = static_cast<const T*>(a.r);
  uint4 xr[RI][CPL], rr[RI][CPL];
#pragma unroll
  for (int g = 0; g < RI; ++g) {
    const int64_t row = row0 + g * RPW;
#pragma unroll
    for (int v = 0; v < CPL; ++v) {
      const int vi = l + LPR * v;
      xr[g][v] = rr[g][v] = make_uint4(0, 0, 0, 0);
      if (row < a.rows && vi < a.nvec) {
        xr[g][v] = ld16raw<true>(X + row * a.x_rs + vi * E);
        if (R) rr[g][v] = ld16raw<true>(R + row * a.r_rs + vi * E);
      }
    }
  }
#pragma unroll
  for (int g = 0; g < RI; ++g) {
    const int64_t row = row0 + g * RPW;
    float f[CPL][E];
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < CPL; ++v) {
      const int vi = l + LPR * v;
      unpack16<T>(xr[g][v], f[v]);
      if (R) {
        float rf[E];
        unpack16<T>(rr[g][v], rf);
#pragma unroll
        for (int e = 0; e < E; ++e)
          f[v][e] = rnd<T>(f[v][e] + (a.alpha == 1.f ? rf[e] : rnd<T>(a.alpha * rf[e])));
      }
      if (vi < a.nvec) {
        if (a.b1) {
          float bf[E];
          load16<T>(static_cast<const T*>(a.b1) + vi * E, bf);
#pragma unroll
          for (int e = 0; e < E; ++e) f[v][e] = rnd<T>(f[v][e] + bf[e]);
        }
        if (a.b2) {
          float bf[E];
          load16<T>(static_cast<const T*>(a.b2) + vi * E, bf);
#pragma unroll
          for (int e = 0; e < E; ++e) f[v][e] = rnd<T>(f[v][e] + bf[e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) f[v][e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < E; ++e) {
        if constexpr (NORM == kNormAda) ss += rnd<T>(f[v][e] * f[v][e]);
        else ss = fmaf(f[v][e], f[v][e], ss);
      }
    }
    if (a.h && row < a.rows) {
#pragma unroll
      for (int v = 0; v < CPL; ++v) {
        const int vi = l + LPR * v;
        if (vi < a.nvec) store16<T>(static_cast<T*>(a.h) + row * a.h_rs + vi * E, f[v]);
      }
    }
    if constexpr (NORM != kNormNone) {
      ss = wave_sum<LPR>(ss);
      float s;
      if constexpr (NORM == kNormAda) {
        const float m = rnd<T>(ss / static_cast<float>(a.dim));
        s = rnd<T>(rsqrtf(rnd<T>(m + a.eps)));
      } else {
        s = rsqrtf(ss / static_cast<float>(a.dim) + a.eps);
      }
      if (row >= a.rows) continue;
#pragma unroll
      for (int v = 0; v < CPL; ++v) {
        const int vi = l + LPR * v;
        if (vi >= a.nvec) continue;
        float wf[E];
        load_elems<WT, E>(static_cast<const WT*>(a.w) + vi * E, wf);
#pragma unroll
        for (int e = 0; e < E; ++e) {
          if constexpr (NORM == kNormAda) f[v][e] = rnd<T>(rnd<T>(f[v][e] * s) * wf[e]);
          else f[v][e] = f[v][e] * s * wf[e];
        }
        store16<T, true>(static_cast<T*>(a.y) + row * a.y_rs + vi * E, f[v]);
      }
    }
  }
}

// Any width / alignment: one wave per row, scalar columns, two passes over
// the row (the first computes the sum of squares, the second re-forms v).
template <typename T, typename WT, int NORM>
__global__ __launch_bounds__(kBlk) void resnorm_scalar_kernel(ResNormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlk / 64) + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const T* X = static_cast<const T*>(a.x) + row * a.x_rs;
  const T* R = a.r ? static_cast<const T*>(a.r) + row * a.r_rs : nullptr;
  const T* B1 = static_cast<const T*>(a.b1);
  const T* B2 = static_cast<const T*>(a.b2);
  auto form = [&](int c) {
    float v = to_f32(X[c]);
    if (R) {
      const float rv = to_f32(R[c]);
      v = rnd<T>(v + (a.alpha == 1.f ? rv : rnd<T>(a.alpha * rv)));
    }
    if (B1) v = rnd<T>(v + to_f32(B1[c]));
    if (B2) v = rnd<T>(v + to_f32(B2[c]));
    return v;
  };
  float ss = 0.f;
  for (int c = lane; c < a.dim; c += 64) {
    const float v = form(c);
    if (a.h) static_cast<T*>(a.h)[row * a.h_rs + c] = from_f32<T>(v);
    if constexpr (NORM == kNormAda) ss += rnd<T>(v * v);
    else ss = fmaf(v, v, ss);
  }
  if constexpr (NORM != kNormNone) {
    ss = wave_sum(ss);
    float s;
    if constexpr (NORM == kNormAda) {
      const float m = rnd<T>(ss / static_cast<float>(a.dim));
      s = rnd<T>(rsqrtf(rnd<T>(m + a.eps)));
    } else {
      s = rsqrtf(ss / static_cast<float>(a.dim) + a.eps);
    }
    const WT* W = static_cast<const WT*>(a.w);
    T* Y = static_cast<T*>(a.y) + row * a.y_rs;
    for (int c = lane; c < a.dim; c += 64) {
      const float v = form(c);
      const float wv = to_f32(W[c]);
      Y[c] = from_f32<T>(NORM == kNormAda ? rnd<T>(v * s) * wv : v * s * wv);
    }
  }
}

template <typename T, typename WT, int LPR, int CPL, int NORM>
int launch_resnorm_vec(const ResNormArgs& a, hipStream_t st) {
  constexpr int RI = CPL >= 4 ? 1 : (CPL >= 2 ? 2 : 4);
  constexpr int RPB = (kBlk / 64) * (64 / LPR) * RI;
  const dim3 grid(static_cast<unsigned>((a.rows + RPB - 1) / RPB));
  resnorm_vec_kernel<T, WT, LPR, CPL, RI, NORM><<<grid, kBlk, 0, st>>>(a);
  return check_launch("resnorm_vec_kernel");
}

template <typename T, typename WT, int NORM>
int launch_resnorm(ResNormArgs a, bool vec_ok, hipStream_t st) {
  constexpr int E = Vec<T>::N;
  if (vec_ok && a.nvec <= 64 * 8) {
    int lpr = 64;
    for (int cand : {64, 32, 16, 8, 4})
      if (a.nvec % cand == 0 && a.nvec / cand <= 8) { lpr = cand; break; }
    const int cpl = (a.nvec + lpr - 1) / lpr;
#define HYDRA_RN_CASE(LP, CP) \
  if (lpr == LP && cpl <= CP) return launch_resnorm_vec<T, WT, LP, CP, NORM>(a, st);
    HYDRA_RN_CASE(4, 1) HYDRA_RN_CASE(4, 2) HYDRA_RN_CASE(4, 4) HYDRA_RN_CASE(4, 8)
    HYDRA_RN_CASE(8, 1) HYDRA_RN_CASE(8, 2) HYDRA_RN_CASE(8, 4) HYDRA_RN_CASE(8, 8)
    HYDRA_RN_CASE(16, 1) HYDRA_RN_CASE(16, 2) HYDRA_RN_CASE(16, 4) HYDRA_RN_CASE(16, 8)
    HYDRA_RN_CASE(32, 1) HYDRA_RN_CASE(32, 2) HYDRA_RN_CASE(32, 4) HYDRA_RN_CASE(32, 8)
    HYDRA_RN_CASE(64, 1) HYDRA_RN_CASE(64, 2) HYDRA_RN_CASE(64, 3) HYDRA_RN_CASE(64, 4)
    HYDRA_RN_CASE(64, 6) HYDRA_RN_CASE(64, 8)
#undef HYDRA_RN_CASE
  }
  (void)E;
  const dim3 grid(static_cast<unsigned>((a.rows + 3) / 4));
  resnorm_scalar_kernel<T, WT, NORM><<<grid, kBlk, 0, st>>>(a);
  return check_launch("resnorm_scalar_kernel");
}

// ---------------------------------------------------------------------------
// MoR executor step for recursion i (mixture_of_recursions.py:449-478), per
// token row with depth d:
//   current = current + rnd(delta * (d >= i))
//   output  = output + rnd(current * (d == i))
// (the straight-through factor (1 + ste_grad) is exactly 1 in the forward).
// In place on current and output.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kBlk) void mor_update_vec_kernel(
    T* __restrict__ cur, const T* __restrict__ delta, T* __restrict__ out,
    const int64_t* __restrict__ depth, uint32_t total, uint32_t cpr, int64_t c_rs,
    int64_t d_rs, int64_t o_rs, int64_t i) {
  constexpr int E = Vec<T>::N;
  const uint32_t t = blockIdx.x * kBlk + threadIdx.x;
  if (t >= total) return;
  const uint32_t r = t / cpr, c = t - r * cpr;
  const int64_t d = depth[r];
  const float act = d >= i ? 1.f : 0.f, ex = d == i ? 1.f : 0.f;
  float cf[E], df[E], of[E];
  T* cp = cur + static_cast<int64_t>(r) * c_rs + c * E;
  T* op = out + static_cast<int64_t>(r) * o_rs + c * E;
  load16<T>(cp, cf);
  load16<T, true>(delta + static_cast<int64_t>(r) * d_rs + c * E, df);
  load16<T>(op, of);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    cf[e] = rnd<T>(cf[e] + df[e] * act);
    of[e] = rnd<T>(of[e] + cf[e] * ex);
  }
  store16<T>(cp, cf);
  store16<T>(op, of);
}

template <typename T>
__global__ __launch_bounds__(kBlk) void mor_update_scalar_kernel(
    T* __restrict__ cur, const T* __restrict__ delta, T* __restrict__ out,
    const int64_t* __restrict__ depth, int64_t total, int64_t dim, int64_t c_rs, int64_t d_rs,
    int64_t o_rs, int64_t i) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlk + threadIdx.x;
  if (t >= total) return;
  const int64_t r = t / dim, c = t - r * dim;
  const int64_t d = depth[r];
  T* cp = cur + r * c_rs + c;
  T* op = out + r * o_rs + c;
  const float cv = rnd<T>(to_f32(*cp) + to_f32(delta[r * d_rs + c]) * (d >= i ? 1.f : 0.f));
  *cp = from_f32<T>(cv);
  *op = from_f32<T>(to_f32(*op) + cv * (d == i ? 1.f : 0.f));
}

// ---------------------------------------------------------------------------
// MoR routing (mixture_of_recursions.py:259-288), per token, each step
// rounded to T as the tensor ops are:
//   l = rnd(rnd(tanh(rnd(logit / 2))) * 3);  p = rnd(sigmoid(l))
//   dc = min_d > 0 ? rnd(min_d + rnd(p * (R - 1 - min_d))) : rnd(p * (R - 1))
//   depth = clamp(round_half_even(dc), min_d, R - 1)
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kBlk) void mor_route_kernel(
    const T* __restrict__ logits, int64_t n, T* __restrict__ probs, T* __restrict__ lout,
    int64_t* __restrict__ depth, int R, int min_d) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlk + threadIdx.x;
  if (t >= n) return;
  const float z = rnd<T>(to_f32(logits[t]) / 2.f);
  const float l = rnd<T>(rnd<T>(tanhf(z)) * 3.f);
  const float p = rnd<T>(1.f / (1.f + expf(-l)));
  float dc;
  if (min_d > 0) dc = rnd<T>(static_cast<float>(min_d) + rnd<T>(p * static_cast<float>(R - 1 - min_d)));
  else dc = rnd<T>(p * static_cast<float>(R - 1));
  int64_t d = static_cast<int64_t>(rintf(dc));  // round half to even, as torch.round
  d = d < min_d ? min_d : (d > R - 1 ? R - 1 : d);
  if (probs) probs[t] = from_f32<T>(p);
  if (lout) lout[t] = from_f32<T>(l);
  depth[t] = d;
}

}  // namespace
}  // namespace hydra

using namespace hydra;

extern "C" int hydra_embedding_fwd(const int64_t* ids, int64_t n, const void* table, int64_t vocab,
                                   int64_t dim, int64_t table_rs, float scale, void* out,
                                   int64_t out_rs, int dtype, void* stream) {
  HYDRA_REQUIRE(n >= 0 && dim >= 1 && vocab >= 1, "embedding: bad size");
  HYDRA_REQUIRE(table_rs >= dim && out_rs >= dim, "embedding: row stride smaller than dim");
  if (n == 0) return HYDRA_OK;
  HYDRA_REQUIRE(ids && table && out, "embedding: null pointer");
  HYDRA_REQUIRE(n * dim / 8 < (int64_t(1) << 31) && n * dim < (int64_t(1) << 40),
                "embedding: too large");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    constexpr int E = Vec<T>::N;
    const int64_t cpr = dim / E;
    const int64_t total = n * cpr;
    const bool vec = dim % E == 0 && table_rs % E == 0 && out_rs % E == 0 && aligned16(table) &&
                     aligned16(out) && total < (int64_t(1) << 31);
    if (vec) {
      embed_vec_kernel<T><<<dim3(static_cast<unsigned>((total + kBlk - 1) / kBlk)), kBlk, 0, st>>>(
          ids, static_cast<const T*>(table), static_cast<T*>(out), (uint32_t)total, (uint32_t)cpr,
          vocab, table_rs, out_rs, scale);
      return check_launch("embed_vec_kernel");
    }
    const int64_t tot = n * dim;
    embed_scalar_kernel<T><<<dim3(static_cast<unsigned>((tot + kBlk - 1) / kBlk)), kBlk, 0, st>>>(
        ids, static_cast<const T*>(table), static_cast<T*>(out), tot, dim, vocab, table_rs, out_rs,
        scale);
    return check_launch("embed_scalar_kernel");
  });
}

extern "C" int hydra_residual_norm_fwd(const void* x, int64_t x_rs, const void* r, int64_t r_rs,
                                       float alpha, const void* b1, const void* b2, const void* w,
                                       float eps, int norm, void* h_out, int64_t h_rs, void* y_out,
                                       int64_t y_rs, int64_t rows, int64_t dim, int dtype,
                                       int w_dtype, void* stream) {
  HYDRA_REQUIRE(rows >= 0 && dim >= 1 && dim <= (int64_t(1) << 30), "residual_norm: bad size");
  HYDRA_REQUIRE(norm == HYDRA_NORM_NONE || norm == HYDRA_NORM_RMS || norm == HYDRA_NORM_ADA,
                "residual_norm: unknown norm mode");
  HYDRA_REQUIRE(x_rs >= dim && (!r || r_rs >= dim) && (!h_out || h_rs >= dim) &&
                    (!y_out || y_rs >= dim),
                "residual_norm: row stride smaller than dim");
  HYDRA_REQUIRE((norm == HYDRA_NORM_NONE) == (y_out == nullptr),
                "residual_norm: y_out is required exactly when a norm is selected");
  HYDRA_REQUIRE(norm == HYDRA_NORM_NONE || w != nullptr, "residual_norm: the norm needs its weight");
  HYDRA_REQUIRE(h_out || y_out, "residual_norm: nothing to write");
  HYDRA_REQUIRE(w_dtype == dtype || w_dtype == HYDRA_F32,
                "residual_norm: the weight must be of x's dtype or fp32");
  HYDRA_REQUIRE((rows + 3) / 4 < (int64_t(1) << 31), "residual_norm: too many rows");
  if (rows == 0) return HYDRA_OK;
  HYDRA_REQUIRE(x != nullptr, "residual_norm: null x");
  auto st = static_cast<hipStream_t>(stream);
  ResNormArgs a{x, x_rs, r, r_rs, alpha, b1, b2, w, h_out, h_rs, y_out, y_rs, rows, 0,
                static_cast<int>(dim), eps};
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    constexpr int E = Vec<T>::N;
    a.nvec = static_cast<int>(dim / E);
    const bool vec = dim % E == 0 && x_rs % E == 0 && (!r || r_rs % E == 0) &&
                     (!h_out || h_rs % E == 0) && (!y_out || y_rs % E == 0) && aligned16(x) &&
                     (!r || aligned16(r)) && (!b1 || aligned16(b1)) && (!b2 || aligned16(b2)) &&
                     (!w || aligned16(w)) && (!h_out || aligned16(h_out)) &&
                     (!y_out || aligned16(y_out));
    auto by_norm = [&](auto wt) -> int {
      using WT = decltype(wt);
      switch (norm) {
        case HYDRA_NORM_RMS: return launch_resnorm<T, WT, kNormRms>(a, vec, st);
        case HYDRA_NORM_ADA: return launch_resnorm<T, WT, kNormAda>(a, vec, st);
        default: return launch_resnorm<T, WT, kNormNone>(a, vec, st);
      }
    };
    if (w_dtype == HYDRA_F32 && !std::is_same<T, float>::value) return by_norm(float());
    return by_norm(T());
  });
}

extern "C" int hydra_mor_update(void* current, int64_t c_rs, const void* delta, int64_t d_rs,
                                void* output, int64_t o_rs, const int64_t* depth, int64_t rows,
                                int64_t dim, int64_t recursion, int dtype, void* stream) {
  HYDRA_REQUIRE(rows >= 0 && dim >= 1, "mor_update: bad size");
  HYDRA_REQUIRE(c_rs >= dim && d_rs >= dim && o_rs >= dim, "mor_update: row stride smaller than dim");
  HYDRA_REQUIRE(recursion >= 0, "mor_update: negative recursion index");
  if (rows == 0) return HYDRA_OK;
  HYDRA_REQUIRE(current && delta && output && depth, "mor_update: null pointer");
  HYDRA_REQUIRE(rows * dim < (int64_t(1) << 40), "mor_update: too large");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    constexpr int E = Vec<T>::N;
    const int64_t cpr = dim / E, total = rows * cpr;
    const bool vec = dim % E == 0 && c_rs % E == 0 && d_rs % E == 0 && o_rs % E == 0 &&
                     aligned16(current) && aligned16(delta) && aligned16(output) &&
                     total < (int64_t(1) << 31);
    if (vec) {
      mor_update_vec_kernel<T><<<dim3(static_cast<unsigned>((total + kBlk - 1) / kBlk)), kBlk, 0, st>>>(
          static_cast<T*>(current), static_cast<const T*>(delta), static_cast<T*>(output), depth,
          (uint32_t)total, (uint32_t)cpr, c_rs, d_rs, o_rs, recursion);
      return check_launch("mor_update_vec_kernel");
    }
    const int64_t tot = rows * dim;
    mor_update_scalar_kernel<T><<<dim3(static_cast<unsigned>((tot + kBlk - 1) / kBlk)), kBlk, 0, st>>>(
        static_cast<T*>(current), static_cast<const T*>(delta), static_cast<T*>(output), depth, tot,
        dim, c_rs, d_rs, o_rs, recursion);
    return check_launch("mor_update_scalar_kernel");
  });
}

extern "C" int hydra_mor_route(const void* logits, int64_t n, void* probs, void* logits_out,
                               int64_t* depth, int64_t n_recursions, int64_t min_depth, int dtype,
                               void* stream) {
  HYDRA_REQUIRE(n >= 0 && n < (int64_t(1) << 40), "mor_route: bad size");
  HYDRA_REQUIRE(n_recursions >= 1 && n_recursions < (int64_t(1) << 20), "mor_route: bad n_recursions");
  HYDRA_REQUIRE(min_depth >= 0 && min_depth <= n_recursions - 1, "mor_route: min_depth out of range");
  if (n == 0) return HYDRA_OK;
  HYDRA_REQUIRE(logits && depth, "mor_route: null pointer");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    mor_route_kernel<T><<<dim3(static_cast<unsigned>((n + kBlk - 1) / kBlk)), kBlk, 0, st>>>(
        static_cast<const T*>(logits), n, static_cast<T*>(probs), static_cast<T*>(logits_out), depth,
        static_cast<int>(n_recursions), static_cast<int>(min_depth));
    return check_launch("mor_route_kernel");
  });
}
