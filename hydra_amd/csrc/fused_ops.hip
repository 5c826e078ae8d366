// Memory-bound fused element ops of hydra/kernels/fused_ops.py, written for
// gfx950: RMSNorm, RoPE, SwiGLU and QK L2-norm.  Each has a 16-byte vector
// path (128-bit global loads/stores, fp32 math, one rounding on store) and a
// scalar path for shapes, strides or alignments the vector path cannot take.
#include "common.h"

#include <algorithm>
#include <mutex>
#include <string>

namespace hydra {

constexpr int kBlock = 256;  // 4 waves

// ===========================================================================
// RMSNorm   (reference: _fused_rms_norm_kernel, fused_ops.py:969-1007)
// LPR lanes per row, CPL 16-byte chunks per lane, RI row groups per wave:
// every lane issues RI*CPL independent 16-byte loads before it reduces, so
// each wave keeps several KB in flight (the kernel is latency- not
// issue-bound otherwise).  The row stays in registers: one read of x, one
// write of y.
// ===========================================================================
template <typename T, int LPR, int CPL, int RI>
__global__ __launch_bounds__(kBlock) void rms_norm_vec_kernel(
    const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ y,
    int64_t rows, int nvec, int dim, int64_t x_rs, int64_t y_rs, float eps) {
  constexpr int E = Vec<T>::N;
  constexpr int RPW = 64 / LPR;                 // rows per wave per group
  constexpr int RPB = (kBlock / 64) * RPW * RI;  // rows per block
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, l = lane % LPR;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * RPB + (wave * RI) * RPW + sub;
  uint4 raw[RI][CPL];
#pragma unroll
  for (int g = 0; g < RI; ++g) {
    const int64_t row = row0 + g * RPW;
#pragma unroll
    for (int v = 0; v < CPL; ++v) {
      const int vi = l + LPR * v;
      raw[g][v] = make_uint4(0, 0, 0, 0);
      if (row < rows && vi < nvec)
        raw[g][v] = ld16raw<true>(x + row * x_rs + vi * E);
    }
  }
#pragma unroll
  for (int g = 0; g < RI; ++g) {
    const int64_t row = row0 + g * RPW;
    float ss = 0.f;
#pragma unroll
    for (int v = 0; v < CPL; ++v) {
      float f[E];
      load16<T>(reinterpret_cast<const T*>(&raw[g][v]), f);
#pragma unroll
      for (int e = 0; e < E; ++e) ss = fmaf(f[e], f[e], ss);
    }
    ss = wave_sum<LPR>(ss);
    const float rinv = rsqrtf(ss / static_cast<float>(dim) + eps);
    if (row >= rows) continue;
#pragma unroll
    for (int v = 0; v < CPL; ++v) {
      const int vi = l + LPR * v;
      if (vi < nvec) {
        float f[E], gw[E];
        load16<T>(reinterpret_cast<const T*>(&raw[g][v]), f);
        load16<T>(w + vi * E, gw);
#pragma unroll
        for (int e = 0; e < E; ++e) f[e] = f[e] * rinv * gw[e];
        store16<T, true>(y + row * y_rs + vi * E, f);
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void rms_norm_scalar_kernel(
    const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ y,
    int64_t rows, int dim, int64_t x_rs, int64_t y_rs, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const T* xr = x + row * x_rs;
  float ss = 0.f;
  for (int i = lane; i < dim; i += 64) {
    const float f = to_f32(xr[i]);
    ss = fmaf(f, f, ss);
  }
  ss = wave_sum(ss);
  const float rinv = rsqrtf(ss / static_cast<float>(dim) + eps);
  T* yr = y + row * y_rs;
  for (int i = lane; i < dim; i += 64) {
    yr[i] = from_f32<T>(to_f32(xr[i]) * rinv * to_f32(w[i]));
  }
}

template <typename T, int LPR, int CPL>
static int launch_rms_vec(const T* X, const T* W, T* Y, int64_t rows, int nvec, int64_t dim,
                          int64_t x_rs, int64_t y_rs, float eps, hipStream_t st) {
  constexpr int RI = CPL >= 4 ? 1 : (CPL >= 2 ? 2 : 4);
  constexpr int RPB = (kBlock / 64) * (64 / LPR) * RI;
  const dim3 grid(static_cast<unsigned>((rows + RPB - 1) / RPB));
  rms_norm_vec_kernel<T, LPR, CPL, RI><<<grid, kBlock, 0, st>>>(X, W, Y, rows, nvec, (int)dim,
                                                               x_rs, y_rs, eps);
  return check_launch("rms_norm_vec_kernel");
}

template <typename T>
static int launch_rms_norm(const void* x, const void* w, void* y, int64_t rows,
                           int64_t dim, int64_t x_rs, int64_t y_rs, float eps,
                           hipStream_t st) {
  constexpr int E = Vec<T>::N;
  const bool vec_ok = dim % E == 0 && x_rs % E == 0 && y_rs % E == 0 &&
                      aligned16(x) && aligned16(w) && aligned16(y);
  const int nvec = static_cast<int>(dim / E);
  auto X = static_cast<const T*>(x);
  auto W = static_cast<const T*>(w);
  auto Y = static_cast<T*>(y);
  if (vec_ok && nvec <= 64 * 8) {
    // Lanes per row: the largest power of two <= 64 that leaves no idle lane
    // slot (nvec % LPR == 0) with at most 8 chunks per lane; else 64 lanes.
    int lpr = 64;
    for (int cand : {64, 32, 16, 8, 4}) {
      if (nvec % cand == 0 && nvec / cand <= 8) { lpr = cand; break; }
    }
    const int cpl = (nvec + lpr - 1) / lpr;
#define HYDRA_RMS_CASE(LP, CP) \
  if (lpr == LP && cpl <= CP) return launch_rms_vec<T, LP, CP>(X, W, Y, rows, nvec, dim, x_rs, y_rs, eps, st);
    HYDRA_RMS_CASE(4, 1) HYDRA_RMS_CASE(4, 2) HYDRA_RMS_CASE(4, 4) HYDRA_RMS_CASE(4, 8)
    HYDRA_RMS_CASE(8, 1) HYDRA_RMS_CASE(8, 2) HYDRA_RMS_CASE(8, 4) HYDRA_RMS_CASE(8, 8)
    HYDRA_RMS_CASE(16, 1) HYDRA_RMS_CASE(16, 2) HYDRA_RMS_CASE(16, 4) HYDRA_RMS_CASE(16, 6) HYDRA_RMS_CASE(16, 8)
    HYDRA_RMS_CASE(32, 1) HYDRA_RMS_CASE(32, 2) HYDRA_RMS_CASE(32, 3) HYDRA_RMS_CASE(32, 4) HYDRA_RMS_CASE(32, 6) HYDRA_RMS_CASE(32, 8)
    HYDRA_RMS_CASE(64, 1) HYDRA_RMS_CASE(64, 2) HYDRA_RMS_CASE(64, 3) HYDRA_RMS_CASE(64, 4) HYDRA_RMS_CASE(64, 6) HYDRA_RMS_CASE(64, 8)
#undef HYDRA_RMS_CASE
  }
  const dim3 grid(static_cast<unsigned>((rows + 3) / 4));
  rms_norm_scalar_kernel<T><<<grid, kBlock, 0, st>>>(X, W, Y, rows, (int)dim, x_rs, y_rs, eps);
  return check_launch("rms_norm_scalar_kernel");
}

// ===========================================================================
// RoPE   (reference: _fused_rope_kernel, fused_ops.py:185-237)
// Output is the contiguous [B,H,S,D] tensor; x may be any strided view.
// BWD: the gradient with respect to x of the same rotation (its transpose:
// sin negated), which the reference's CPU path gets from autograd.
// 16-byte path (rope_hg_kernel): a thread rotates one chunk (E/2 pairs) of
// HB heads of one row.  Otherwise (rope_scalar_kernel) blockIdx.y + 65535
// blockIdx.z = b*H + h and a thread rotates one pair.
// ===========================================================================
template <typename T, typename C, bool BWD>
__global__ __launch_bounds__(kBlock) void rope_scalar_kernel(
    const T* __restrict__ x, const C* __restrict__ cs, const C* __restrict__ sn,
    T* __restrict__ out, int BH, int H, int S, int D, int64_t xb, int64_t xh, int64_t xsr,
    int64_t xd, int64_t cs_rs) {
  const int half = D / 2;
  const int bh = blockIdx.y + 65535 * blockIdx.z;
  if (bh >= BH) return;
  const int b = bh / H, h = bh - b * H;
  const int t = blockIdx.x * kBlock + threadIdx.x;
  const int s = t / half;
  if (s >= S) return;
  const int p = t - s * half;
  const T* xr = x + b * xb + h * xh + static_cast<int64_t>(s) * xsr;
  const float x1 = to_f32(xr[(2 * p) * xd]), x2 = to_f32(xr[(2 * p + 1) * xd]);
  const float cv = to_f32(cs[static_cast<int64_t>(s) * cs_rs + p]);
  const float sv = BWD ? -to_f32(sn[static_cast<int64_t>(s) * cs_rs + p]) : to_f32(sn[static_cast<int64_t>(s) * cs_rs + p]);
  T* o = out + (static_cast<int64_t>(bh) * S + s) * D;
  o[2 * p] = from_f32<T>(x1 * cv - x2 * sv);
  o[2 * p + 1] = from_f32<T>(x1 * sv + x2 * cv);
}

// Thread (b, group of HB heads, s, chunk c): the cos/sin chunk is read once
// and applied to HB heads, whose loads are all issued first.  At
// [8,12,2048,64] bf16: one head per thread 11.1 us, HB 4 10.7 us, HB 6 with
// 128-thread blocks 9.7 us (the cos/sin reads, which hit L2, fall from 1/2
// to 1/6 of the HBM bytes and each thread keeps 6 loads in flight).
// E/2 consecutive cos (or sin) values as one aligned vector load.
template <typename C, int N>
struct alignas(N * sizeof(C)) CsVec { C v[N]; };

// Grid: x over (s, c) of one (b, head group), y + 65535 z = b * ng + hg, so
// a thread finds its row with one 32-bit shift (or division) and no 64-bit
// index arithmetic; csh = log2(D / E) when that is a power of two, else -1.
template <typename T, typename C, int HB, int BS, bool CSV, bool BWD>
__global__ __launch_bounds__(BS) void rope_hg_kernel(
    const T* __restrict__ x, const C* __restrict__ cs, const C* __restrict__ sn,
    T* __restrict__ out, int H, int S, int D, int64_t xb, int64_t xh, int64_t xsr,
    int64_t cs_rs, int nbg, int csh) {
  constexpr int E = Vec<T>::N;
  const int bg = blockIdx.y + 65535 * blockIdx.z;
  const int cpr = D / E;
  const int t = blockIdx.x * BS + threadIdx.x;
  if (bg >= nbg || t >= S * cpr) return;
  const int s = csh >= 0 ? t >> csh : t / cpr;
  const int c = t - s * cpr;
  const int ng = (H + HB - 1) / HB;
  const int64_t b = bg / ng;
  const int hg = bg - static_cast<int>(b) * ng;
  const int h0 = hg * HB;
  uint4 raw[HB];
  const T* xr = x + b * xb + static_cast<int64_t>(s) * xsr + c * E;
#pragma unroll
  for (int j = 0; j < HB; ++j)
    if (h0 + j < H) raw[j] = ld16raw<true>(xr + (h0 + j) * xh);
  float cv[E / 2], sv[E / 2];
  const C* cr = cs + static_cast<int64_t>(s) * cs_rs + c * (E / 2);
  const C* sr = sn + static_cast<int64_t>(s) * cs_rs + c * (E / 2);
  if constexpr (CSV) {
    const CsVec<C, E / 2> cw = *reinterpret_cast<const CsVec<C, E / 2>*>(cr);
    const CsVec<C, E / 2> sw = *reinterpret_cast<const CsVec<C, E / 2>*>(sr);
#pragma unroll
    for (int p = 0; p < E / 2; ++p) {
      cv[p] = to_f32(cw.v[p]);
      sv[p] = BWD ? -to_f32(sw.v[p]) : to_f32(sw.v[p]);
    }
  } else {
#pragma unroll
    for (int p = 0; p < E / 2; ++p) {
      cv[p] = to_f32(cr[p]);
      sv[p] = BWD ? -to_f32(sr[p]) : to_f32(sr[p]);
    }
  }
  T* orow = out + (b * H * S + s) * D + c * E;
#pragma unroll
  for (int j = 0; j < HB; ++j) {
    if (h0 + j >= H) continue;
    float f[E], o[E];
    unpack16<T>(raw[j], f);
#pragma unroll
    for (int p = 0; p < E / 2; ++p) {
      const float x1 = f[2 * p], x2 = f[2 * p + 1];
      o[2 * p] = x1 * cv[p] - x2 * sv[p];
      o[2 * p + 1] = x1 * sv[p] + x2 * cv[p];
    }
    store16<T, true>(orow + static_cast<int64_t>(h0 + j) * S * D, o);
  }
}

template <typename T, typename C, bool BWD>
static int launch_rope(const void* x, const void* cs, const void* sn, void* out,
                       int64_t B, int64_t H, int64_t S, int64_t D,
                       const int64_t* xs, int64_t cs_rs, hipStream_t st) {
  constexpr int E = Vec<T>::N;
  auto X = static_cast<const T*>(x);
  auto CS = static_cast<const C*>(cs);
  auto SN = static_cast<const C*>(sn);
  auto O = static_cast<T*>(out);
  const bool vec_ok = xs[3] == 1 && D % E == 0 && xs[0] % E == 0 &&
                      xs[1] % E == 0 && xs[2] % E == 0 && aligned16(x) &&
                      aligned16(out);
  constexpr int kRopeBlock = 128;
  const int hb = H % 6 == 0 ? 6 : 4;
  const int64_t nbg = B * ((H + hb - 1) / hb);
  const int64_t per_bg = S * (D / E);
  if (vec_ok && per_bg < (int64_t(1) << 31) - kRopeBlock) {  // nbg <= B * H < 2^31
    const dim3 grid(static_cast<unsigned>((per_bg + kRopeBlock - 1) / kRopeBlock),
                    static_cast<unsigned>(std::min<int64_t>(nbg, 65535)),
                    static_cast<unsigned>((nbg + 65534) / 65535));
    const int cpr = static_cast<int>(D / E);
    const int csh = (cpr & (cpr - 1)) == 0 ? __builtin_ctz(static_cast<unsigned>(cpr)) : -1;
    constexpr size_t kCsBytes = (E / 2) * sizeof(C);
    const bool csv = cs_rs % (E / 2) == 0 && reinterpret_cast<uintptr_t>(cs) % kCsBytes == 0 &&
                     reinterpret_cast<uintptr_t>(sn) % kCsBytes == 0;
#define HYDRA_ROPE_CASE(HB, CV)                                                            \
  if (hb == HB && csv == CV)                                                               \
    rope_hg_kernel<T, C, HB, kRopeBlock, CV, BWD><<<grid, kRopeBlock, 0, st>>>(            \
        X, CS, SN, O, (int)H, (int)S, (int)D, xs[0], xs[1], xs[2], cs_rs, (int)nbg, csh);
    HYDRA_ROPE_CASE(6, true) HYDRA_ROPE_CASE(6, false) HYDRA_ROPE_CASE(4, true) HYDRA_ROPE_CASE(4, false)
#undef HYDRA_ROPE_CASE
    return check_launch("rope_hg_kernel");
  }
  const int64_t threads = S * (D / 2);
  const dim3 grid(static_cast<unsigned>((threads + kBlock - 1) / kBlock),
                  static_cast<unsigned>(std::min<int64_t>(B * H, 65535)),
                  static_cast<unsigned>((B * H + 65534) / 65535));
  rope_scalar_kernel<T, C, BWD><<<grid, kBlock, 0, st>>>(X, CS, SN, O, (int)(B * H), (int)H, (int)S,
                                                    (int)D, xs[0], xs[1], xs[2],
                                                    xs[3], cs_rs);
  return check_launch("rope_scalar_kernel");
}

// ===========================================================================
// SwiGLU   (reference: _fused_swiglu_kernel, fused_ops.py:703-725)
// gate/up are read straight from the two halves of the gate_up GEMM output,
// so no contiguous copies are made.  silu(g) = g / (1 + exp(-g)).
// ===========================================================================
// silu(g) = g / (1 + exp(-g)) with the hardware reciprocal (1 ulp) in place
// of an IEEE division: the division's fix-up sequence made the kernel
// VALU-bound (40.8 -> 34.4 us at C2); the result is rounded to the storage
// type right after, so the difference is at the fp32 ulp level.
__device__ __forceinline__ float silu_f32(float g) { return g * __builtin_amdgcn_rcpf(1.f + __expf(-g)); }

template <typename T, int U>
__global__ __launch_bounds__(kBlock) void swiglu_vec_kernel(
    const T* __restrict__ g, const T* __restrict__ u, T* __restrict__ o,
    uint32_t total, uint32_t cpr, int64_t g_rs, int64_t u_rs, int64_t o_rs) {
  constexpr int E = Vec<T>::N;
  const uint32_t base = (blockIdx.x * U) * kBlock + threadIdx.x;
  float gf[U][E], uf[U][E];
  uint32_t rr[U], cc[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t idx = base + j * kBlock;
    rr[j] = idx / cpr;
    cc[j] = idx - rr[j] * cpr;
    if (idx < total) {
      load16<T, true>(g + rr[j] * g_rs + cc[j] * E, gf[j]);
      load16<T, true>(u + rr[j] * u_rs + cc[j] * E, uf[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t idx = base + j * kBlock;
    if (idx < total) {
      float of[E];
#pragma unroll
      for (int e = 0; e < E; ++e) of[e] = silu_f32(gf[j][e]) * uf[j][e];
      store16<T, true>(o + rr[j] * o_rs + cc[j] * E, of);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void swiglu_scalar_kernel(
    const T* __restrict__ g, const T* __restrict__ u, T* __restrict__ o,
    int64_t total, int64_t hidden, int64_t g_rs, int64_t u_rs, int64_t o_rs) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (idx >= total) return;
  const int64_t r = idx / hidden, c = idx - r * hidden;
  o[r * o_rs + c] = from_f32<T>(silu_f32(to_f32(g[r * g_rs + c])) * to_f32(u[r * u_rs + c]));
}

template <typename T>
static int launch_swiglu(const void* g, const void* u, void* o, int64_t rows,
                         int64_t hidden, int64_t g_rs, int64_t u_rs, int64_t o_rs,
                         hipStream_t st) {
  constexpr int E = Vec<T>::N;
  constexpr int U = 2;
  auto G = static_cast<const T*>(g);
  auto Up = static_cast<const T*>(u);
  auto O = static_cast<T*>(o);
  const int64_t cpr = hidden / E;
  const int64_t total_vec = rows * cpr;
  const bool vec_ok = hidden % E == 0 && g_rs % E == 0 && u_rs % E == 0 &&
                      o_rs % E == 0 && aligned16(g) && aligned16(u) && aligned16(o) &&
                      total_vec < (int64_t(1) << 31);
  if (vec_ok) {
    const dim3 grid(static_cast<unsigned>((total_vec + U * kBlock - 1) / (U * kBlock)));
    swiglu_vec_kernel<T, U><<<grid, kBlock, 0, st>>>(G, Up, O, (uint32_t)total_vec,
                                                     (uint32_t)cpr, g_rs, u_rs, o_rs);
    return check_launch("swiglu_vec_kernel");
  }
  const int64_t total = rows * hidden;
  const dim3 grid(static_cast<unsigned>((total + kBlock - 1) / kBlock));
  swiglu_scalar_kernel<T><<<grid, kBlock, 0, st>>>(G, Up, O, total, hidden, g_rs,
                                                   u_rs, o_rs);
  return check_launch("swiglu_scalar_kernel");
}

// ===========================================================================
// QK L2-norm   (reference: _fused_qk_norm_kernel, fused_ops.py:323-369)
// LPR lanes per row, one 16-byte chunk each; rows of q then rows of k.
// ===========================================================================
template <typename T, int LPR>
__global__ __launch_bounds__(kBlock) void qk_norm_vec_kernel(
    const T* __restrict__ q, const T* __restrict__ k, T* __restrict__ qo,
    T* __restrict__ ko, int64_t q_rows, int64_t k_rows, float scale, float temp) {
  constexpr int E = Vec<T>::N;
  constexpr int HD = LPR * E;
  const int64_t gt = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  int64_t row = gt / LPR;
  const int c = static_cast<int>(gt % LPR);
  const bool is_k = row >= q_rows;
  if (is_k) row -= q_rows;
  const bool live = is_k ? row < k_rows : true;
  const T* src = is_k ? k : q;
  T* dst = is_k ? ko : qo;
  float f[E];
  float ss = 0.f;
  if (live) {
    load16<T>(src + row * HD + c * E, f);
#pragma unroll
    for (int e = 0; e < E; ++e) ss = fmaf(f[e], f[e], ss);
  }
  ss = wave_sum<LPR>(ss);
  if (!live) return;
  float fac = rsqrtf(ss + 1e-8f) * scale;
  if (is_k) fac *= temp;
#pragma unroll
  for (int e = 0; e < E; ++e) f[e] *= fac;
  store16<T>(dst + row * HD + c * E, f);
}

template <typename T>
__global__ __launch_bounds__(kBlock) void qk_norm_scalar_kernel(
    const T* __restrict__ q, const T* __restrict__ k, T* __restrict__ qo,
    T* __restrict__ ko, int64_t q_rows, int64_t k_rows, int hd, float scale,
    float temp) {
  int64_t row = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const bool is_k = row >= q_rows;
  if (is_k) row -= q_rows;
  if (is_k && row >= k_rows) return;
  const T* src = (is_k ? k : q) + row * hd;
  T* dst = (is_k ? ko : qo) + row * hd;
  float ss = 0.f;
  for (int i = 0; i < hd; ++i) {
    const float f = to_f32(src[i]);
    ss = fmaf(f, f, ss);
  }
  float fac = rsqrtf(ss + 1e-8f) * scale;
  if (is_k) fac *= temp;
  for (int i = 0; i < hd; ++i) dst[i] = from_f32<T>(to_f32(src[i]) * fac);
}

template <typename T>
static int launch_qk_norm(const void* q, const void* k, void* qo, void* ko,
                          int64_t q_rows, int64_t k_rows, int64_t hd, float scale,
                          float temp, hipStream_t st) {
  constexpr int E = Vec<T>::N;
  auto Q = static_cast<const T*>(q);
  auto K = static_cast<const T*>(k);
  auto QO = static_cast<T*>(qo);
  auto KO = static_cast<T*>(ko);
  const int64_t lpr = hd / E;
  const bool vec_ok = hd % E == 0 && lpr >= 1 && lpr <= 64 && (lpr & (lpr - 1)) == 0 &&
                      aligned16(q) && aligned16(k) && aligned16(qo) && aligned16(ko);
  if (vec_ok) {
    const int64_t threads = (q_rows + k_rows) * lpr;
    const dim3 grid(static_cast<unsigned>((threads + kBlock - 1) / kBlock));
#define HYDRA_QKN_CASE(L)                                                      \
  case L:                                                                      \
    qk_norm_vec_kernel<T, L><<<grid, kBlock, 0, st>>>(Q, K, QO, KO, q_rows,    \
                                                      k_rows, scale, temp);    \
    return check_launch("qk_norm_vec_kernel");
    switch (lpr) {
      HYDRA_QKN_CASE(1) HYDRA_QKN_CASE(2) HYDRA_QKN_CASE(4) HYDRA_QKN_CASE(8)
      HYDRA_QKN_CASE(16) HYDRA_QKN_CASE(32) HYDRA_QKN_CASE(64)
      default: break;
    }
#undef HYDRA_QKN_CASE
  }
  const dim3 grid(static_cast<unsigned>((q_rows + k_rows + kBlock - 1) / kBlock));
  qk_norm_scalar_kernel<T><<<grid, kBlock, 0, st>>>(Q, K, QO, KO, q_rows, k_rows,
                                                    (int)hd, scale, temp);
  return check_launch("qk_norm_scalar_kernel");
}

// ===========================================================================
// Backward of the fused ops (reference: the PyTorch backward paths of
// fused_ops.py, which the Triton backward kernels follow): fp32 math, the
// +-100 clamp, one rounding to the input dtype on store.
// ===========================================================================

// RMSNorm backward (reference: _rms_norm_backward_pytorch,
// fused_ops.py:1251-1281; _fused_rms_norm_backward_kernel :1027-1111).  Per
// row, r = rsqrt(mean(x^2) + eps), xn = x * r, corr = mean(g * w * xn),
// grad_x = clamp(g * w * r - xn * corr) -- the reference's correction term,
// as written.  The weight gradient sum over rows of xn * g is folded into
// the same pass: each lane keeps the sums of its columns over the block's
// rows, the block reduces them through LDS and writes one fp32 partial row;
// rms_norm_bwd_w_kernel adds the partial rows in a fixed order
// (deterministic) and clamps.  The block walks rows
// [blockIdx.x * RPB + i * gridDim.x * RPB, ..), RI row groups per wave per
// step with all their loads issued first.
template <typename T, typename WT, int LPR, int CPL, int RI>
__global__ __launch_bounds__(kBlock) void rms_norm_bwd_kernel(
    const T* __restrict__ x, const WT* __restrict__ w, const T* __restrict__ gy,
    T* __restrict__ gx, float* __restrict__ part, int64_t rows, int nvec, int dim,
    int64_t x_rs, int64_t gy_rs, int64_t gx_rs, float eps) {
  constexpr int E = Vec<T>::N;
  constexpr int RPW = 64 / LPR;                   // rows per wave per group
  constexpr int RPB = (kBlock / 64) * RPW * RI;   // rows per block step
  __shared__ float red[kBlock / 64][RPW][CPL * E * LPR];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / LPR, l = lane % LPR;
  float wf[CPL][E];
  float accw[CPL][E];
#pragma unroll
  for (int v = 0; v < CPL; ++v) {
    const int vi = l + LPR * v;
#pragma unroll
    for (int e = 0; e < E; ++e) accw[v][e] = 0.f;
    if (vi < nvec) {
#pragma unroll
      for (int q = 0; q < E * int(sizeof(WT)) / 16; ++q)
        load16<WT>(w + vi * E + q * (16 / int(sizeof(WT))), wf[v] + q * (16 / int(sizeof(WT))));
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) wf[v][e] = 0.f;
    }
  }
  for (int64_t rb = static_cast<int64_t>(blockIdx.x) * RPB; rb < rows;
       rb += static_cast<int64_t>(gridDim.x) * RPB) {
    // the RI row groups' loads are all issued before any reduction
    float xf[RI][CPL][E], gf[RI][CPL][E];
#pragma unroll
    for (int g = 0; g < RI; ++g) {
      const int64_t row = rb + (wave * RI + g) * RPW + sub;
#pragma unroll
      for (int v = 0; v < CPL; ++v) {
        const int vi = l + LPR * v;
        if (row < rows && vi < nvec) {
          load16<T, true>(x + row * x_rs + vi * E, xf[g][v]);
          load16<T, true>(gy + row * gy_rs + vi * E, gf[g][v]);
        } else {
#pragma unroll
          for (int e = 0; e < E; ++e) xf[g][v][e] = gf[g][v][e] = 0.f;
        }
      }
    }
#pragma unroll
    for (int g = 0; g < RI; ++g) {
      const int64_t row = rb + (wave * RI + g) * RPW + sub;
      float ss = 0.f;
#pragma unroll
      for (int v = 0; v < CPL; ++v)
#pragma unroll
        for (int e = 0; e < E; ++e) ss = fmaf(xf[g][v][e], xf[g][v][e], ss);
      ss = wave_sum<LPR>(ss);
      const float r = rsqrtf(ss / static_cast<float>(dim) + eps);
      float cs = 0.f;
#pragma unroll
      for (int v = 0; v < CPL; ++v)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const float xn = xf[g][v][e] * r;
          cs = fmaf(gf[g][v][e] * wf[v][e], xn, cs);
          accw[v][e] = fmaf(xn, gf[g][v][e], accw[v][e]);
        }
      const float corr = wave_sum<LPR>(cs) / static_cast<float>(dim);
      if (row >= rows) continue;
#pragma unroll
      for (int v = 0; v < CPL; ++v) {
        const int vi = l + LPR * v;
        if (vi >= nvec) continue;
        float o[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
          const float xn = xf[g][v][e] * r;
          o[e] = fminf(fmaxf(gf[g][v][e] * wf[v][e] * r - xn * corr, -100.f), 100.f);
        }
        store16<T, true>(gx + row * gx_rs + vi * E, o);
      }
    }
  }
  // Weight-gradient partial of this block: sum over (wave, sub) in order.
#pragma unroll
  for (int v = 0; v < CPL; ++v)
#pragma unroll
    for (int e = 0; e < E; ++e) red[wave][sub][(v * LPR + l) * E + e] = accw[v][e];
  __syncthreads();
  for (int c = threadIdx.x; c < CPL * E * LPR; c += kBlock) {
    // c = (v * LPR + l) * E + e  <->  column (l + LPR * v) * E + e
    const int e = c % E, vl = c / E, v = vl / LPR, ll = vl - v * LPR;
    const int col = (ll + LPR * v) * E + e;
    if (col >= dim) continue;
    float s = 0.f;
    for (int wv = 0; wv < kBlock / 64; ++wv)
      for (int sb = 0; sb < RPW; ++sb) s += red[wv][sb][c];
    part[static_cast<int64_t>(blockIdx.x) * dim + col] = s;
  }
}

// Weight gradient from the n partial rows, in one launch: a block of 1024
// threads per 32-column strip (each row segment one 128-byte line), thread
// (c, g) adding partial rows g, g + 32, .. of column c in order (8 loads in
// flight), then the 32 sums of each column in order through LDS; clamped.
// Deterministic.  After the main kernel: 19.9 us for both launches at
// [16384, 768] against 22.5 with 64-column strips of 16 waves (12 blocks).
constexpr int kRmsBwdCols = 32;
constexpr int kRmsBwdGroups = 1024 / kRmsBwdCols;
template <typename GT>
__global__ __launch_bounds__(1024) void rms_norm_bwd_w_kernel(const float* __restrict__ part,
                                                             GT* __restrict__ gw, int n, int dim) {
  constexpr int U = 8;
  __shared__ float red[kRmsBwdGroups][kRmsBwdCols];
  const int c = threadIdx.x % kRmsBwdCols, grp = threadIdx.x / kRmsBwdCols;
  const int col = blockIdx.x * kRmsBwdCols + c;
  float s = 0.f;
  if (col < dim) {
    int r = grp;
    for (; r + kRmsBwdGroups * (U - 1) < n; r += kRmsBwdGroups * U) {
      float a[U];
#pragma unroll
      for (int u = 0; u < U; ++u) a[u] = part[static_cast<int64_t>(r + kRmsBwdGroups * u) * dim + col];
#pragma unroll
      for (int u = 0; u < U; ++u) s += a[u];
    }
    for (; r < n; r += kRmsBwdGroups) s += part[static_cast<int64_t>(r) * dim + col];
  }
  red[grp][c] = s;
  __syncthreads();
  if (threadIdx.x < kRmsBwdCols && col < dim) {
    float t = 0.f;
#pragma unroll 8
    for (int g = 0; g < kRmsBwdGroups; ++g) t += red[g][c];
    gw[col] = from_f32<GT>(fminf(fmaxf(t, -100.f), 100.f));
  }
}

// Rows of any width / alignment: one wave per row, scalar columns.
template <typename T, typename WT>
__global__ __launch_bounds__(kBlock) void rms_norm_bwd_scalar_kernel(
    const T* __restrict__ x, const WT* __restrict__ w, const T* __restrict__ gy,
    T* __restrict__ gx, float* __restrict__ part, int64_t rows, int dim, int64_t x_rs,
    int64_t gy_rs, int64_t gx_rs, float eps) {
  // part [gridDim.x * 4][dim]: one partial row per wave (wave-private, so
  // no reduction step); rms_norm_bwd_w_kernel adds them in order.
  const int lane = threadIdx.x & 63;
  const int64_t wid = static_cast<int64_t>(blockIdx.x) * (kBlock / 64) + (threadIdx.x >> 6);
  const int64_t nw = static_cast<int64_t>(gridDim.x) * (kBlock / 64);
  float* pw = part + wid * dim;
  for (int c = lane; c < dim; c += 64) pw[c] = 0.f;
  for (int64_t row = wid; row < rows; row += nw) {
    const T* xr = x + row * x_rs;
    const T* gr = gy + row * gy_rs;
    float ss = 0.f;
    for (int c = lane; c < dim; c += 64) {
      const float f = to_f32(xr[c]);
      ss = fmaf(f, f, ss);
    }
    const float r = rsqrtf(wave_sum(ss) / static_cast<float>(dim) + eps);
    float cs = 0.f;
    for (int c = lane; c < dim; c += 64)
      cs = fmaf(to_f32(gr[c]) * to_f32(w[c]), to_f32(xr[c]) * r, cs);
    const float corr = wave_sum(cs) / static_cast<float>(dim);
    for (int c = lane; c < dim; c += 64) {
      const float xn = to_f32(xr[c]) * r, g = to_f32(gr[c]);
      gx[row * gx_rs + c] = from_f32<T>(fminf(fmaxf(g * to_f32(w[c]) * r - xn * corr, -100.f), 100.f));
      pw[c] = fmaf(xn, g, pw[c]);
    }
  }
}

// The weight gradient from the n partial rows.
template <typename GT>
static int rms_bwd_reduce_w(const float* part, GT* gw, int n, int dim, hipStream_t st) {
  const int rc0 = check_launch("rms_norm_bwd_kernel");
  if (rc0 != HYDRA_OK) return rc0;
  rms_norm_bwd_w_kernel<GT><<<dim3((dim + kRmsBwdCols - 1) / kRmsBwdCols), 1024, 0, st>>>(part, gw, n, dim);
  return check_launch("rms_norm_bwd_w_kernel");
}

// Partial rows of the weight gradient (fp32 [n][dim]) the two backward
// paths write: at most kRmsBwdParts rows for any shape.  768 = 3 resident
// 4-wave blocks on each of 256 CUs at 144 VGPRs (dim 768 bf16): one full
// wave of blocks, no tail (512 blocks of two row groups: 18.1 us, 768 of
// one: 16.7 us; 896 and 1024 blocks, which do not all fit at once: 20 us).
constexpr int kRmsBwdParts = 768;

template <typename T, typename WT, int LPR, int CPL>
static int launch_rms_bwd_vec(const T* X, const WT* W, const T* GY, T* GX, WT* GW, float* part,
                              int64_t rows, int nvec, int dim, int64_t x_rs, int64_t gy_rs,
                              int64_t gx_rs, float eps, hipStream_t st) {
  constexpr int RI = CPL >= 3 ? 1 : (CPL == 2 ? 2 : 4);  // row groups per wave per step
  constexpr int RPB = (kBlock / 64) * (64 / LPR) * RI;
  // A fixed number of blocks (from the shape only), so the summation order
  // of the weight gradient does not depend on the device.
  const int nblk = static_cast<int>(std::min<int64_t>((rows + RPB - 1) / RPB, kRmsBwdParts));
  rms_norm_bwd_kernel<T, WT, LPR, CPL, RI><<<dim3(nblk), kBlock, 0, st>>>(X, W, GY, GX, part, rows, nvec, dim,
                                                                     x_rs, gy_rs, gx_rs, eps);
  return rms_bwd_reduce_w(part, GW, nblk, dim, st);
}

// part: fp32 scratch of at least kRmsBwdParts * dim elements.
template <typename T, typename WT>
static int launch_rms_norm_bwd(const void* x, const void* w, const void* gy, void* gx, void* gw,
                               float* part, int64_t rows, int64_t dim, int64_t x_rs, int64_t gy_rs,
                               int64_t gx_rs, float eps, hipStream_t st) {
  constexpr int E = Vec<T>::N;
  auto X = static_cast<const T*>(x);
  auto W = static_cast<const WT*>(w);
  auto GY = static_cast<const T*>(gy);
  auto GX = static_cast<T*>(gx);
  auto GW = static_cast<WT*>(gw);
  const bool vec_ok = dim % E == 0 && x_rs % E == 0 && gy_rs % E == 0 && gx_rs % E == 0 && aligned16(x) &&
                      aligned16(w) && aligned16(gy) && aligned16(gx);
  const int nvec = static_cast<int>(dim / E);
  if (vec_ok && nvec <= 64 * 4) {
    int lpr = 64;
    for (int cand : {64, 32, 16, 8, 4}) {
      if (nvec % cand == 0 && nvec / cand <= 4) {
        lpr = cand;
        break;
      }
    }
    const int cpl = (nvec + lpr - 1) / lpr;
#define HYDRA_RMSB_CASE(LP, CP)                                                                           \
  if (lpr == LP && cpl <= CP)                                                                             \
    return launch_rms_bwd_vec<T, WT, LP, CP>(X, W, GY, GX, GW, part, rows, nvec, (int)dim, x_rs, gy_rs, gx_rs, \
                                             eps, st);
    HYDRA_RMSB_CASE(4, 1) HYDRA_RMSB_CASE(4, 2) HYDRA_RMSB_CASE(4, 4)
    HYDRA_RMSB_CASE(8, 1) HYDRA_RMSB_CASE(8, 2) HYDRA_RMSB_CASE(8, 4)
    HYDRA_RMSB_CASE(16, 1) HYDRA_RMSB_CASE(16, 2) HYDRA_RMSB_CASE(16, 4)
    HYDRA_RMSB_CASE(32, 1) HYDRA_RMSB_CASE(32, 2) HYDRA_RMSB_CASE(32, 3) HYDRA_RMSB_CASE(32, 4)
    HYDRA_RMSB_CASE(64, 1) HYDRA_RMSB_CASE(64, 2) HYDRA_RMSB_CASE(64, 3) HYDRA_RMSB_CASE(64, 4)
#undef HYDRA_RMSB_CASE
  }
  const int nblk = static_cast<int>(std::min<int64_t>((rows + 3) / 4, kRmsBwdParts / 4));
  rms_norm_bwd_scalar_kernel<T, WT><<<dim3(nblk), kBlock, 0, st>>>(X, W, GY, GX, part, rows, (int)dim, x_rs,
                                                                  gy_rs, gx_rs, eps);
  return rms_bwd_reduce_w(part, GW, nblk * 4, (int)dim, st);
}

// SwiGLU backward (reference: _swiglu_backward_pytorch, fused_ops.py:926-948;
// _fused_swiglu_backward_kernel :748-805): s = sigmoid(g),
// grad_gate = clamp(go * u * s * (1 + g * (1 - s))), grad_up = clamp(go * g * s).
__device__ __forceinline__ float sigmoid_f32(float g) { return __builtin_amdgcn_rcpf(1.f + __expf(-g)); }

template <typename T, int U>
__global__ __launch_bounds__(kBlock) void swiglu_bwd_vec_kernel(
    const T* __restrict__ g, const T* __restrict__ u, const T* __restrict__ gy, T* __restrict__ gg,
    T* __restrict__ gu, uint32_t total, uint32_t cpr, int64_t g_rs, int64_t u_rs, int64_t gy_rs,
    int64_t gg_rs, int64_t gu_rs) {
  constexpr int E = Vec<T>::N;
  const uint32_t base = (blockIdx.x * U) * kBlock + threadIdx.x;
  float gf[U][E], uf[U][E], of[U][E];
  uint32_t rr[U], cc[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t idx = base + j * kBlock;
    rr[j] = idx / cpr;
    cc[j] = idx - rr[j] * cpr;
    if (idx < total) {
      load16<T, true>(g + rr[j] * g_rs + cc[j] * E, gf[j]);
      load16<T, true>(u + rr[j] * u_rs + cc[j] * E, uf[j]);
      load16<T, true>(gy + rr[j] * gy_rs + cc[j] * E, of[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t idx = base + j * kBlock;
    if (idx >= total) continue;
    float a[E], b[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float x = gf[j][e], s = sigmoid_f32(x);
      a[e] = fminf(fmaxf(of[j][e] * uf[j][e] * (s * (1.f + x * (1.f - s))), -100.f), 100.f);
      b[e] = fminf(fmaxf(of[j][e] * (x * s), -100.f), 100.f);
    }
    store16<T, true>(gg + rr[j] * gg_rs + cc[j] * E, a);
    store16<T, true>(gu + rr[j] * gu_rs + cc[j] * E, b);
  }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void swiglu_bwd_scalar_kernel(
    const T* __restrict__ g, const T* __restrict__ u, const T* __restrict__ gy, T* __restrict__ gg,
    T* __restrict__ gu, int64_t total, int64_t hidden, int64_t g_rs, int64_t u_rs, int64_t gy_rs,
    int64_t gg_rs, int64_t gu_rs) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (idx >= total) return;
  const int64_t r = idx / hidden, c = idx - r * hidden;
  const float x = to_f32(g[r * g_rs + c]), up = to_f32(u[r * u_rs + c]), o = to_f32(gy[r * gy_rs + c]);
  const float s = sigmoid_f32(x);
  gg[r * gg_rs + c] = from_f32<T>(fminf(fmaxf(o * up * (s * (1.f + x * (1.f - s))), -100.f), 100.f));
  gu[r * gu_rs + c] = from_f32<T>(fminf(fmaxf(o * (x * s), -100.f), 100.f));
}

template <typename T>
static int launch_swiglu_bwd(const void* g, const void* u, const void* gy, void* gg, void* gu, int64_t rows,
                             int64_t hidden, int64_t g_rs, int64_t u_rs, int64_t gy_rs, int64_t gg_rs,
                             int64_t gu_rs, hipStream_t st) {
  constexpr int E = Vec<T>::N;
  constexpr int U = 2;
  auto G = static_cast<const T*>(g);
  auto Up = static_cast<const T*>(u);
  auto GY = static_cast<const T*>(gy);
  auto GG = static_cast<T*>(gg);
  auto GU = static_cast<T*>(gu);
  const int64_t cpr = hidden / E;
  const int64_t total_vec = rows * cpr;
  const bool vec_ok = hidden % E == 0 && g_rs % E == 0 && u_rs % E == 0 && gy_rs % E == 0 && gg_rs % E == 0 &&
                      gu_rs % E == 0 && aligned16(g) && aligned16(u) && aligned16(gy) && aligned16(gg) &&
                      aligned16(gu) && total_vec < (int64_t(1) << 31);
  if (vec_ok) {
    const dim3 grid(static_cast<unsigned>((total_vec + U * kBlock - 1) / (U * kBlock)));
    swiglu_bwd_vec_kernel<T, U><<<grid, kBlock, 0, st>>>(G, Up, GY, GG, GU, (uint32_t)total_vec, (uint32_t)cpr,
                                                         g_rs, u_rs, gy_rs, gg_rs, gu_rs);
    return check_launch("swiglu_bwd_vec_kernel");
  }
  const int64_t total = rows * hidden;
  const dim3 grid(static_cast<unsigned>((total + kBlock - 1) / kBlock));
  swiglu_bwd_scalar_kernel<T><<<grid, kBlock, 0, st>>>(G, Up, GY, GG, GU, total, hidden, g_rs, u_rs, gy_rs,
                                                       gg_rs, gu_rs);
  return check_launch("swiglu_bwd_scalar_kernel");
}

// QK-norm backward (reference: _qk_norm_backward_pytorch, fused_ops.py:638-672;
// _fused_qk_norm_backward_kernel :389-471): per row n = max(||x||, 1e-6),
// xn = x / n, grad = clamp(s / n * (g - xn * <xn, g>)), s = scale (q) or
// scale * temperature (k).  Rows of q then rows of k, contiguous.
template <typename T, int LPR>
__global__ __launch_bounds__(kBlock) void qk_norm_bwd_vec_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ gqo, const T* __restrict__ gko,
    T* __restrict__ gq, T* __restrict__ gk, int64_t q_rows, int64_t k_rows, float scale, float temp) {
  constexpr int E = Vec<T>::N;
  constexpr int HD = LPR * E;
  const int64_t gt = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  int64_t row = gt / LPR;
  const int c = static_cast<int>(gt % LPR);
  const bool is_k = row >= q_rows;
  if (is_k) row -= q_rows;
  const bool live = is_k ? row < k_rows : true;
  float f[E], g[E];
  float ss = 0.f, dot = 0.f;
  if (live) {
    load16<T>((is_k ? k : q) + row * HD + c * E, f);
    load16<T>((is_k ? gko : gqo) + row * HD + c * E, g);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      ss = fmaf(f[e], f[e], ss);
      dot = fmaf(f[e], g[e], dot);
    }
  }
  ss = wave_sum<LPR>(ss);
  dot = wave_sum<LPR>(dot);
  if (!live) return;
  const float ninv = 1.f / fmaxf(__builtin_sqrtf(ss), 1e-6f);
  const float d = dot * ninv;  // <xn, g>
  const float fac = (is_k ? scale * temp : scale) * ninv;
  float o[E];
#pragma unroll
  for (int e = 0; e < E; ++e) o[e] = fminf(fmaxf(fac * (g[e] - f[e] * ninv * d), -100.f), 100.f);
  store16<T>((is_k ? gk : gq) + row * HD + c * E, o);
}

template <typename T>
__global__ __launch_bounds__(kBlock) void qk_norm_bwd_scalar_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ gqo, const T* __restrict__ gko,
    T* __restrict__ gq, T* __restrict__ gk, int64_t q_rows, int64_t k_rows, int hd, float scale, float temp) {
  int64_t row = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const bool is_k = row >= q_rows;
  if (is_k) row -= q_rows;
  if (is_k && row >= k_rows) return;
  const T* xr = (is_k ? k : q) + row * hd;
  const T* gr = (is_k ? gko : gqo) + row * hd;
  T* dst = (is_k ? gk : gq) + row * hd;
  float ss = 0.f, dot = 0.f;
  for (int i = 0; i < hd; ++i) {
    const float f = to_f32(xr[i]);
    ss = fmaf(f, f, ss);
    dot = fmaf(f, to_f32(gr[i]), dot);
  }
  const float ninv = 1.f / fmaxf(__builtin_sqrtf(ss), 1e-6f);
  const float d = dot * ninv;
  const float fac = (is_k ? scale * temp : scale) * ninv;
  for (int i = 0; i < hd; ++i)
    dst[i] = from_f32<T>(fminf(fmaxf(fac * (to_f32(gr[i]) - to_f32(xr[i]) * ninv * d), -100.f), 100.f));
}

template <typename T>
static int launch_qk_norm_bwd(const void* q, const void* k, const void* gqo, const void* gko, void* gq,
                              void* gk, int64_t q_rows, int64_t k_rows, int64_t hd, float scale, float temp,
                              hipStream_t st) {
  constexpr int E = Vec<T>::N;
  auto Q = static_cast<const T*>(q);
  auto K = static_cast<const T*>(k);
  auto GQO = static_cast<const T*>(gqo);
  auto GKO = static_cast<const T*>(gko);
  auto GQ = static_cast<T*>(gq);
  auto GK = static_cast<T*>(gk);
  const int64_t lpr = hd / E;
  const bool vec_ok = hd % E == 0 && lpr >= 1 && lpr <= 64 && (lpr & (lpr - 1)) == 0 && aligned16(q) &&
                      aligned16(k) && aligned16(gqo) && aligned16(gko) && aligned16(gq) && aligned16(gk);
  if (vec_ok) {
    const int64_t threads = (q_rows + k_rows) * lpr;
    const dim3 grid(static_cast<unsigned>((threads + kBlock - 1) / kBlock));
#define HYDRA_QKNB_CASE(L)                                                                              \
  case L:                                                                                               \
    qk_norm_bwd_vec_kernel<T, L><<<grid, kBlock, 0, st>>>(Q, K, GQO, GKO, GQ, GK, q_rows, k_rows, scale, \
                                                          temp);                                        \
    return check_launch("qk_norm_bwd_vec_kernel");
    switch (lpr) {
      HYDRA_QKNB_CASE(1) HYDRA_QKNB_CASE(2) HYDRA_QKNB_CASE(4) HYDRA_QKNB_CASE(8)
      HYDRA_QKNB_CASE(16) HYDRA_QKNB_CASE(32) HYDRA_QKNB_CASE(64)
      default: break;
    }
#undef HYDRA_QKNB_CASE
  }
  const dim3 grid(static_cast<unsigned>((q_rows + k_rows + kBlock - 1) / kBlock));
  qk_norm_bwd_scalar_kernel<T><<<grid, kBlock, 0, st>>>(Q, K, GQO, GKO, GQ, GK, q_rows, k_rows, (int)hd, scale,
                                                        temp);
  return check_launch("qk_norm_bwd_scalar_kernel");
}

}  // namespace hydra

using namespace hydra;

extern "C" int hydra_rms_norm_fwd(const void* x, const void* w, void* y,
                                  int64_t rows, int64_t dim, int64_t x_rs,
                                  int64_t y_rs, float eps, int dtype, void* stream) {
  HYDRA_REQUIRE(rows >= 0 && dim >= 1, "rms_norm: rows must be >= 0 and dim >= 1");
  HYDRA_REQUIRE(dim <= (int64_t(1) << 30), "rms_norm: dim too large");
  HYDRA_REQUIRE(x_rs >= dim && y_rs >= dim, "rms_norm: row stride smaller than dim");
  if (rows == 0) return HYDRA_OK;
  HYDRA_REQUIRE(x && w && y, "rms_norm: null pointer");
  HYDRA_REQUIRE((rows + 3) / 4 < (int64_t(1) << 31), "rms_norm: too many rows");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    return launch_rms_norm<T>(x, w, y, rows, dim, x_rs, y_rs, eps, st);
  });
}

extern "C" int hydra_rope_fwd(const void* x, const void* cos, const void* sin,
                              void* out, int64_t B, int64_t H, int64_t S, int64_t D,
                              const int64_t* xs, int64_t cs_rs, int dtype,
                              int cs_dtype, void* stream) {
  HYDRA_REQUIRE(B >= 0 && H >= 0 && S >= 0 && D >= 0, "rope: negative size");
  HYDRA_REQUIRE(D % 2 == 0, "rope: head_dim must be even");
  HYDRA_REQUIRE(xs != nullptr, "rope: null stride array");
  if (B * H * S * D == 0) return HYDRA_OK;
  HYDRA_REQUIRE(x && cos && sin && out, "rope: null pointer");
  HYDRA_REQUIRE(cs_rs >= D / 2, "rope: cos/sin row stride smaller than head_dim/2");
  HYDRA_REQUIRE(B * H < (int64_t(1) << 31), "rope: B*H too large");
  HYDRA_REQUIRE(S * D < (int64_t(1) << 31), "rope: S*D too large");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    switch (cs_dtype) {
      case HYDRA_F32: return launch_rope<T, float, false>(x, cos, sin, out, B, H, S, D, xs, cs_rs, st);
      case HYDRA_BF16: return launch_rope<T, bf16, false>(x, cos, sin, out, B, H, S, D, xs, cs_rs, st);
      case HYDRA_F16: return launch_rope<T, f16, false>(x, cos, sin, out, B, H, S, D, xs, cs_rs, st);
      default: return fail(HYDRA_ERR_ARG, "rope: unknown cos/sin dtype code");
    }
  });
}

extern "C" int hydra_swiglu_fwd(const void* gate, const void* up, void* out,
                                int64_t rows, int64_t hidden, int64_t g_rs,
                                int64_t u_rs, int64_t o_rs, int dtype, void* stream) {
  HYDRA_REQUIRE(rows >= 0 && hidden >= 0, "swiglu: negative size");
  if (rows * hidden == 0) return HYDRA_OK;
  HYDRA_REQUIRE(gate && up && out, "swiglu: null pointer");
  HYDRA_REQUIRE(g_rs >= hidden && u_rs >= hidden && o_rs >= hidden,
                "swiglu: row stride smaller than hidden");
  HYDRA_REQUIRE((rows * hidden + kBlock - 1) / kBlock < (int64_t(1) << 31),
                "swiglu: tensor too large");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    return launch_swiglu<T>(gate, up, out, rows, hidden, g_rs, u_rs, o_rs, st);
  });
}

extern "C" int hydra_qk_norm_fwd(const void* q, const void* k, void* q_out,
                                 void* k_out, int64_t q_rows, int64_t k_rows,
                                 int64_t hd, float scale, float temperature,
                                 int dtype, void* stream) {
  HYDRA_REQUIRE(q_rows >= 0 && k_rows >= 0 && hd >= 1, "qk_norm: bad size");
  if (q_rows + k_rows == 0) return HYDRA_OK;
  HYDRA_REQUIRE((q_rows == 0 || (q && q_out)) && (k_rows == 0 || (k && k_out)),
                "qk_norm: null pointer");
  HYDRA_REQUIRE((q_rows + k_rows) * hd < (int64_t(1) << 40), "qk_norm: tensor too large");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    return launch_qk_norm<T>(q, k, q_out, k_out, q_rows, k_rows, hd, scale,
                             temperature, st);
  });
}

// The shared body of the RMSNorm backward entry points: argument checks, the
// zero-row case, and the dtype dispatch with the weight-gradient partials
// in `part` (kRmsBwdParts * dim fp32).
static int rms_norm_bwd_body(const void* x, const void* w, const void* grad_y, void* grad_x,
                             void* grad_w, float* part, int64_t rows, int64_t dim, int64_t x_rs,
                             int64_t gy_rs, int64_t gx_rs, float eps, int dtype, int w_dtype,
                             hipStream_t st) {
  if (rows == 0) {
    // no rows: the weight gradient is zero (a fill kernel, not a memset, so
    // the call can sit in a captured graph)
    return HYDRA_DISPATCH_DTYPE(w_dtype, GT, [&] {
      rms_norm_bwd_w_kernel<GT><<<dim3(static_cast<unsigned>((dim + kRmsBwdCols - 1) / kRmsBwdCols)), 1024, 0, st>>>(
          nullptr, static_cast<GT*>(grad_w), 0, static_cast<int>(dim));
      return check_launch("rms_norm_bwd_w_kernel");
    });
  }
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    if (w_dtype == HYDRA_F32 && !std::is_same<T, float>::value)
      return launch_rms_norm_bwd<T, float>(x, w, grad_y, grad_x, grad_w, part, rows, dim, x_rs, gy_rs,
                                           gx_rs, eps, st);
    return launch_rms_norm_bwd<T, T>(x, w, grad_y, grad_x, grad_w, part, rows, dim, x_rs, gy_rs, gx_rs,
                                     eps, st);
  });
}

static int rms_norm_bwd_check(const void* x, const void* w, const void* grad_y, void* grad_x,
                              void* grad_w, int64_t rows, int64_t dim, int64_t x_rs, int64_t gy_rs,
                              int64_t gx_rs, int dtype, int w_dtype) {
  HYDRA_REQUIRE(rows >= 0 && dim >= 1, "rms_norm_bwd: rows must be >= 0 and dim >= 1");
  HYDRA_REQUIRE(dim <= (int64_t(1) << 24), "rms_norm_bwd: dim too large");
  HYDRA_REQUIRE(x_rs >= dim && gy_rs >= dim && gx_rs >= dim, "rms_norm_bwd: row stride smaller than dim");
  HYDRA_REQUIRE(x && w && grad_y && grad_x && grad_w, "rms_norm_bwd: null pointer");
  HYDRA_REQUIRE(dtype_size(dtype) > 0, "rms_norm_bwd: unknown dtype code");
  HYDRA_REQUIRE(w_dtype == dtype || w_dtype == HYDRA_F32,
                "rms_norm_bwd: the weight must be of x's dtype or fp32");
  return HYDRA_OK;
}

// ---- allocation-free variant ----------------------------------------------
// hydra_rms_norm_bwd_noalloc keeps the weight-gradient partial rows in this
// file-scope device array instead of caller-provided scratch, so
// the call allocates nothing.  12 MiB per device (kRmsBwdParts rows of up to
// kNoAllocMaxDim fp32), held until the process ends.  Every partial row the
// reduction reads is written earlier in the same call, so nothing has to be
// cleared between calls; calls that overlap on one device share the array and
// race.
constexpr int64_t kNoAllocMaxDim = 4096;
static __device__ __align__(256) float scratch[kRmsBwdParts * kNoAllocMaxDim];

// The device address of `scratch` on the current device, looked up once per
// device (each device holds its own copy of the array).  In host code the
// name `scratch` is only a handle for the runtime, never an address.
static int noalloc_scratch(float** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static float* ptrs[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(HYDRA_ERR_LAUNCH, "rms_norm_bwd_noalloc: no usable current device");
  std::lock_guard<std::mutex> lock(mu);
  if (ptrs[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(HYDRA_ERR_LAUNCH, std::string("rms_norm_bwd_noalloc: hipGetSymbolAddress failed: ") +
                                        hipGetErrorString(e));
    ptrs[dev] = static_cast<float*>(p);
  }
  *out = ptrs[dev];
  return HYDRA_OK;
}

extern "C" int hydra_rms_norm_bwd_noalloc(const void* x, const void* w, const void* grad_y, void* grad_x,
                                          void* grad_w, int64_t rows, int64_t dim, int64_t x_rs,
                                          int64_t gy_rs, int64_t gx_rs, float eps, int dtype, int w_dtype,
                                          void* stream) {
  const int rc = rms_norm_bwd_check(x, w, grad_y, grad_x, grad_w, rows, dim, x_rs, gy_rs, gx_rs, dtype,
                                    w_dtype);
  if (rc != HYDRA_OK) return rc;
  if (dim > kNoAllocMaxDim)
    return fail(HYDRA_ERR_ARG, "rms_norm_bwd_noalloc: dim " + std::to_string(dim) +
                                   " exceeds the fixed scratch's maximum of " +
                                   std::to_string(kNoAllocMaxDim) + "; use hydra_rms_norm_bwd");
  float* part = nullptr;
  const int src = noalloc_scratch(&part);
  if (src != HYDRA_OK) return src;
  return rms_norm_bwd_body(x, w, grad_y, grad_x, grad_w, part, rows, dim, x_rs, gy_rs, gx_rs, eps, dtype,
                           w_dtype, static_cast<hipStream_t>(stream));
}

extern "C" int64_t hydra_rms_norm_bwd_workspace(int64_t rows, int64_t dim) {
  if (rows <= 0 || dim <= 0) return 0;
  return static_cast<int64_t>(kRmsBwdParts) * dim * static_cast<int64_t>(sizeof(float));
}

extern "C" int hydra_rms_norm_bwd(const void* x, const void* w, const void* grad_y, void* grad_x,
                                  void* grad_w, int64_t rows, int64_t dim, int64_t x_rs, int64_t gy_rs,
                                  int64_t gx_rs, float eps, int dtype, int w_dtype, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  const int rc = rms_norm_bwd_check(x, w, grad_y, grad_x, grad_w, rows, dim, x_rs, gy_rs, gx_rs, dtype,
                                    w_dtype);
  if (rc != HYDRA_OK) return rc;
  const int64_t need = hydra_rms_norm_bwd_workspace(rows, dim);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return fail(HYDRA_ERR_ARG, "rms_norm_bwd: workspace of " + std::to_string(need) +
                                   " bytes required (hydra_rms_norm_bwd_workspace)");
  return rms_norm_bwd_body(x, w, grad_y, grad_x, grad_w, static_cast<float*>(workspace), rows, dim, x_rs,
                           gy_rs, gx_rs, eps, dtype, w_dtype, static_cast<hipStream_t>(stream));
}

extern "C" int hydra_rope_bwd(const void* grad_y, const void* cos, const void* sin, void* grad_x,
                              int64_t B, int64_t H, int64_t S, int64_t D, const int64_t* gys, int64_t cs_rs,
                              int dtype, int cs_dtype, void* stream) {
  HYDRA_REQUIRE(B >= 0 && H >= 0 && S >= 0 && D >= 0, "rope_bwd: negative size");
  HYDRA_REQUIRE(D % 2 == 0, "rope_bwd: head_dim must be even");
  HYDRA_REQUIRE(gys != nullptr, "rope_bwd: null stride array");
  if (B * H * S * D == 0) return HYDRA_OK;
  HYDRA_REQUIRE(grad_y && cos && sin && grad_x, "rope_bwd: null pointer");
  HYDRA_REQUIRE(cs_rs >= D / 2, "rope_bwd: cos/sin row stride smaller than head_dim/2");
  HYDRA_REQUIRE(B * H < (int64_t(1) << 31), "rope_bwd: B*H too large");
  HYDRA_REQUIRE(S * D < (int64_t(1) << 31), "rope_bwd: S*D too large");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    switch (cs_dtype) {
      case HYDRA_F32: return launch_rope<T, float, true>(grad_y, cos, sin, grad_x, B, H, S, D, gys, cs_rs, st);
      case HYDRA_BF16: return launch_rope<T, bf16, true>(grad_y, cos, sin, grad_x, B, H, S, D, gys, cs_rs, st);
      case HYDRA_F16: return launch_rope<T, f16, true>(grad_y, cos, sin, grad_x, B, H, S, D, gys, cs_rs, st);
      default: return fail(HYDRA_ERR_ARG, "rope_bwd: unknown cos/sin dtype code");
    }
  });
}

extern "C" int hydra_swiglu_bwd(const void* gate, const void* up, const void* grad_y, void* grad_gate,
                                void* grad_up, int64_t rows, int64_t hidden, int64_t g_rs, int64_t u_rs,
                                int64_t gy_rs, int64_t gg_rs, int64_t gu_rs, int dtype, void* stream) {
  HYDRA_REQUIRE(rows >= 0 && hidden >= 0, "swiglu_bwd: negative size");
  if (rows * hidden == 0) return HYDRA_OK;
  HYDRA_REQUIRE(gate && up && grad_y && grad_gate && grad_up, "swiglu_bwd: null pointer");
  HYDRA_REQUIRE(g_rs >= hidden && u_rs >= hidden && gy_rs >= hidden && gg_rs >= hidden && gu_rs >= hidden,
                "swiglu_bwd: row stride smaller than hidden");
  HYDRA_REQUIRE((rows * hidden + kBlock - 1) / kBlock < (int64_t(1) << 31), "swiglu_bwd: tensor too large");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    return launch_swiglu_bwd<T>(gate, up, grad_y, grad_gate, grad_up, rows, hidden, g_rs, u_rs, gy_rs, gg_rs,
                                gu_rs, st);
  });
}

extern "C" int hydra_qk_norm_bwd(const void* q, const void* k, const void* grad_qo, const void* grad_ko,
                                 void* grad_q, void* grad_k, int64_t q_rows, int64_t k_rows, int64_t hd,
                                 float scale, float temperature, int dtype, void* stream) {
  HYDRA_REQUIRE(q_rows >= 0 && k_rows >= 0 && hd >= 1, "qk_norm_bwd: bad size");
  if (q_rows + k_rows == 0) return HYDRA_OK;
  HYDRA_REQUIRE((q_rows == 0 || (q && grad_qo && grad_q)) && (k_rows == 0 || (k && grad_ko && grad_k)),
                "qk_norm_bwd: null pointer");
  HYDRA_REQUIRE((q_rows + k_rows) * hd < (int64_t(1) << 40), "qk_norm_bwd: tensor too large");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    return launch_qk_norm_bwd<T>(q, k, grad_qo, grad_ko, grad_q, grad_k, q_rows, k_rows, hd, scale, temperature,
                                 st);
  });
}
