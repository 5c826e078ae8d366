// Cross-entropy rows of the chunked LM-head loss on gfx950.
// Reference semantics: chunked_cross_entropy / ChunkedCrossEntropyFunction
// (hydra/kernels/fused_ops.py:1303-1379, 1382-1531): per token row of logits
// x[0..V), with target t (ignore_index rows contribute nothing; other
// targets are clamped to [0, V), :1407-1422),
//   loss_row = logsumexp(x) - x[t],
// and for the backward (:1459-1531), grad_x = (softmax(x) - onehot(t)) * scale
// with scale = grad_output / n_valid, and zero rows for ignored tokens.
// The projections around it (logits = h W^T, grad_h = grad_x W,
// grad_W = grad_x^T h) are plain GEMMs and stay on hipBLASLt.
//
// One 256-thread workgroup per row: an online (max, sum-exp) pass with
// 16-byte loads, a workgroup reduction, then (backward) the row rewritten
// in place.  HBM-bound: a row is read once and written once -- rows of up to
// 32 16-byte chunks per thread (vocab <= 32768 fp32 / 65536 bf16) are held
// in registers between the two phases, longer rows are read a second time.
#include "common.h"

namespace hydra {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// (m, s) with s = sum exp2(x - m), merged.
__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
  const float mx = fmaxf(m, m2);
  if (mx == -INFINITY) return;  // both empty
  s = s * __builtin_amdgcn_exp2f(m - mx) + s2 * __builtin_amdgcn_exp2f(m2 - mx);
  m = mx;
}

template <typename T, bool VEC, bool GRAD>
__global__ __launch_bounds__(256) void ce_rows_kernel(
    const T* logits, int64_t rs, const int64_t* __restrict__ targets,  // logits may alias grad
    float* __restrict__ loss, float* __restrict__ lse_out, T* grad, int64_t grs,
    const float* __restrict__ grad_scale, int V, int64_t ignore_index) {
  constexpr int E = VEC ? 16 / int(sizeof(T)) : 1;
  __shared__ float red_m[4], red_s[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const T* x = logits + row * rs;
  // Pass 1: online max / sum of exp2 over the row, in log2 units.
  float m = -INFINITY, s = 0.f;
  for (int e = tid * E; e < V; e += 256 * E) {
    float v[E];
    // Streamed once when no gradient pass follows: non-temporal loads.
    if constexpr (VEC) load16<T, !GRAD>(x + e, v);
    else v[0] = to_f32(x[e]);
    float cm = v[0] * kLog2e;
#pragma unroll
    for (int i = 1; i < E; ++i) cm = fmaxf(cm, v[i] * kLog2e);
    if (cm == -INFINITY) continue;  // all -inf: adds nothing (and exp2(-inf + inf) is NaN)
    float cs = 0.f;
#pragma unroll
    for (int i = 0; i < E; ++i) cs += __builtin_amdgcn_exp2f(fmaf(v[i], kLog2e, -cm));
    lse_merge(m, s, cm, cs);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off), s2 = __shfl_xor(s, off);
    lse_merge(m, s, m2, s2);
  }
  // x[t] is read before the barrier: with grad == logits, other threads
  // overwrite the row after it.
  const int64_t t_raw = targets[row];
  const bool valid = t_raw != ignore_index;
  const int t = static_cast<int>(t_raw < 0 ? 0 : (t_raw >= V ? V - 1 : t_raw));
  const float xt = tid == 0 ? to_f32(x[t]) : 0.f;
  if (lane == 0) { red_m[wave] = m; red_s[wave] = s; }
  __syncthreads();
  m = red_m[0];
  s = red_s[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) lse_merge(m, s, red_m[w], red_s[w]);
  const float lse2 = m + __log2f(s);  // log2-domain logsumexp
  if (tid == 0) {
    loss[row] = valid ? (lse2 - xt * kLog2e) * kLn2 : 0.f;
    if (lse_out) lse_out[row] = lse2 * kLn2;
  }
  if constexpr (GRAD) {
    // Pass 2: grad = (softmax - onehot(t)) * scale; ignored rows get zeros.
    // In place is allowed (grad == logits): each element is read before
    // the same thread writes it.
    const float sc = valid ? *grad_scale : 0.f;
    T* g = grad + row * grs;
    for (int e = tid * E; e < V; e += 256 * E) {
      float v[E];
      if constexpr (VEC) load16<T>(x + e, v);
      else v[0] = to_f32(x[e]);
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float p = __builtin_amdgcn_exp2f(fmaf(v[i], kLog2e, -lse2));
        v[i] = (p - (e + i == t ? 1.f : 0.f)) * sc;
      }
      if constexpr (VEC) store16<T>(g + e, v);
      else g[e] = from_f32<T>(v[0]);
    }
  }
}

// Gradient variant for rows that fit in registers (V <= 256 * NCH * E):
// the row is read from HBM once, kept in VGPRs across the reduction, and
// rewritten from there.
template <typename T, int NCH>
__global__ __launch_bounds__(256) void ce_rows_reg_kernel(
    const T* logits, int64_t rs, const int64_t* __restrict__ targets,  // logits may alias grad
    float* __restrict__ loss, float* __restrict__ lse_out, T* grad, int64_t grs,
    const float* __restrict__ grad_scale, int V, int64_t ignore_index) {
  constexpr int E = 16 / int(sizeof(T));
  __shared__ float red_m[4], red_s[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const T* x = logits + row * rs;
  // The row's chunks stay in registers as loaded (16-bit types packed: 128
  // VGPRs at 32 chunks, where unpacked floats would spill) and are widened
  // where used.
  uint4 raw[NCH];
  auto chunk = [&](int c, float (&f)[E]) {
    const int e = (c * 256 + tid) * E;
    if (e < V) {
      load16<T>(reinterpret_cast<const T*>(&raw[c]), f);
    } else {
#pragma unroll
      for (int i = 0; i < E; ++i) f[i] = -INFINITY;
    }
  };
  float m = -INFINITY, s = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e = (c * 256 + tid) * E;
    raw[c] = e < V ? ld16raw<true>(x + e) : make_uint4(0, 0, 0, 0);  // read once: non-temporal
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    float v[E];
    chunk(c, v);
    float cm = v[0] * kLog2e;
#pragma unroll
    for (int i = 1; i < E; ++i) cm = fmaxf(cm, v[i] * kLog2e);
    if (cm == -INFINITY) continue;
    float cs = 0.f;
#pragma unroll
    for (int i = 0; i < E; ++i) cs += __builtin_amdgcn_exp2f(fmaf(v[i], kLog2e, -cm));
    lse_merge(m, s, cm, cs);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off), s2 = __shfl_xor(s, off);
    lse_merge(m, s, m2, s2);
  }
  // x[t] is read before the barrier: with grad == logits, other threads
  // overwrite the row after it.
  const int64_t t_raw = targets[row];
  const bool valid = t_raw != ignore_index;
  const int t = static_cast<int>(t_raw < 0 ? 0 : (t_raw >= V ? V - 1 : t_raw));
  const float xt = tid == 0 ? to_f32(x[t]) : 0.f;
  if (lane == 0) { red_m[wave] = m; red_s[wave] = s; }
  __syncthreads();
  m = red_m[0];
  s = red_s[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) lse_merge(m, s, red_m[w], red_s[w]);
  const float lse2 = m + __log2f(s);
  if (tid == 0) {
    loss[row] = valid ? (lse2 - xt * kLog2e) * kLn2 : 0.f;
    if (lse_out) lse_out[row] = lse2 * kLn2;
  }
  const float sc = valid ? *grad_scale : 0.f;
  T* g = grad + row * grs;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int e = (c * 256 + tid) * E;
    if (e < V) {
      float v[E], o[E];
      chunk(c, v);
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float p = __builtin_amdgcn_exp2f(fmaf(v[i], kLog2e, -lse2));
        o[i] = (p - (e + i == t ? 1.f : 0.f)) * sc;
      }
      store16<T, true>(g + e, o);
    }
  }
}

template <typename T, bool GRAD>
int launch(const void* logits, int64_t rs, const int64_t* targets, float* loss, float* lse,
           void* grad, int64_t grs, const float* scale, int64_t rows, int V, int64_t ignore,
           hipStream_t st) {
  constexpr int E = 16 / int(sizeof(T));
  const bool vec = V % E == 0 && rs % E == 0 && aligned16(logits) &&
                   (!GRAD || (grs % E == 0 && aligned16(grad)));
  const dim3 grid(static_cast<unsigned>(rows));
  const T* x = static_cast<const T*>(logits);
  T* g = static_cast<T*>(grad);
  if constexpr (GRAD) {
    // Register-resident rows: up to 32 chunks of 16 bytes per thread.
    const int nch = (V / E + 255) / 256;
    if (vec && nch <= 32) {
#define HYDRA_CE_REG(N) \
  ce_rows_reg_kernel<T, N><<<grid, 256, 0, st>>>(x, rs, targets, loss, lse, g, grs, scale, V, ignore)
      if (nch <= 8) HYDRA_CE_REG(8);
      else if (nch <= 16) HYDRA_CE_REG(16);
      else HYDRA_CE_REG(32);
#undef HYDRA_CE_REG
      return check_launch("ce_rows");
    }
  }
  if (vec)
    ce_rows_kernel<T, true, GRAD><<<grid, 256, 0, st>>>(x, rs, targets, loss, lse, g, grs, scale, V, ignore);
  else
    ce_rows_kernel<T, false, GRAD><<<grid, 256, 0, st>>>(x, rs, targets, loss, lse, g, grs, scale, V, ignore);
  return check_launch("ce_rows");
}

}  // namespace
}  // namespace hydra

using namespace hydra;

extern "C" int hydra_ce_rows(const void* logits, int64_t rows, int64_t vocab, int64_t logits_rs,
                             const int64_t* targets, int64_t ignore_index, float* loss,
                             float* lse, void* grad, int64_t grad_rs, const float* grad_scale,
                             int dtype, void* stream) {
  HYDRA_REQUIRE(rows >= 0 && vocab >= 1, "ce_rows: bad size");
  HYDRA_REQUIRE(vocab < (int64_t(1) << 31) && rows < (int64_t(1) << 31), "ce_rows: too large");
  HYDRA_REQUIRE(logits_rs >= vocab && (!grad || grad_rs >= vocab), "ce_rows: row stride < vocab");
  HYDRA_REQUIRE(dtype == HYDRA_F32 || dtype == HYDRA_BF16 || dtype == HYDRA_F16,
                "ce_rows: unknown dtype");
  if (rows == 0) return HYDRA_OK;
  HYDRA_REQUIRE(logits && targets && loss, "ce_rows: null pointer");
  HYDRA_REQUIRE(!grad || grad_scale, "ce_rows: the gradient needs grad_scale");
  auto st = static_cast<hipStream_t>(stream);
  const int V = static_cast<int>(vocab);
#define HYDRA_CE(T)                                                                                  \
  return grad ? launch<T, true>(logits, logits_rs, targets, loss, lse, grad, grad_rs, grad_scale,   \
                                rows, V, ignore_index, st)                                          \
              : launch<T, false>(logits, logits_rs, targets, loss, lse, grad, grad_rs, grad_scale,  \
                                 rows, V, ignore_index, st)
  switch (dtype) {
    case HYDRA_F32: HYDRA_CE(float);
    case HYDRA_BF16: HYDRA_CE(bf16);
    default: HYDRA_CE(f16);
  }
#undef HYDRA_CE
}
