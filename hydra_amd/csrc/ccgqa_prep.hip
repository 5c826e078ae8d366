// CCGQA q/k/v preparation on gfx950: everything of CCGQAAttention.forward
// between the fused qkv GEMM and the attention core, for one tile of TT
// tokens of one batch row per workgroup
// (reference: hydra/attention/backends/ccgqa/attention.py:205-266 and
// OptimizedConvSequence.forward, kernels/fused_conv.py:39-62):
//
//   q0|k0|v_curr|v_prev = qkv[s]                       (split, :205-216)
//   v[s] = v_curr[s] | v_prev[s-1] (0 at s=0)          (value shift, :211-220)
//   y1 = conv1(pad2(q0)), groups = heads, k=3          (fused_conv.py:52-53)
//   y2 = conv2(pad2(y1)), dense, k=3                   (fused_conv.py:56-57)
//   QK-mean from the pre-conv q0/k0                    (:224-246)
//   q = normalize(q); k = normalize(k) * temperature   (:260-262)
//   q, k = rope(q), rope(k)                            (:264-266)
//
// The tile stages the qkv rows of tokens [s0-4, s0+TT) (two k=3 causal convs
// reach 4 tokens back) in LDS.  Every value the reference materialises as a
// tensor of the working dtype (conv outputs, means, sums, the norm, the
// normalised vector, the temperature product, the rotated output) is rounded
// to that dtype at the same point, so the result tracks the reference's
// rounding sequence and not just its mathematics.
//
// Conv weights come tap-major, [3][out][in/groups] (PyTorch's Conv1d weight
// [out, in/groups, 3] permuted (2, 0, 1)), so a row of input channels for one
// (tap, output channel) is contiguous.
//
// Two variants: ccgqa_prep_mfma_kernel (bf16, head_dim in {16, 32, 64, 128}) runs
// both convs as v_mfma_f32_32x32x16_bf16 tiles over LDS-staged token rows;
// ccgqa_prep_generic_kernel (VALU, fp32 arithmetic) takes every other case.
#include "common.h"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace hydra {

// Tiles whose epilogue gave up waiting for the QK-mean terms (see
// ccgqa_prep_mfma_kernel); read by hydra_ccgqa_prep_faults.  Stays 0 unless
// the hardware or the compiler breaks the kernel's forward-progress
// assumptions.
__device__ unsigned int g_prep_wait_faults = 0;

template <typename T>
__device__ __forceinline__ float rnd(float v) {
  return to_f32(from_f32<T>(v));
}

// Eight values rounded to bf16 in place, two per v_cvt_pk_bf16_f32.
__device__ __forceinline__ void rnd8(float* v) {
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const uint32_t p = pack2<bf16>(v[e], v[e + 1]);
    v[e] = __uint_as_float(p << 16);
    v[e + 1] = __uint_as_float(p & 0xffff0000u);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void ccgqa_prep_generic_kernel(
    const T* __restrict__ qkv, int64_t qkv_rs, const T* __restrict__ wq1,
    const T* __restrict__ wq2, const T* __restrict__ wk1, const T* __restrict__ wk2,
    const T* __restrict__ temp, const float* __restrict__ cs, const float* __restrict__ sn,
    int64_t cs_rs, T* __restrict__ qo, T* __restrict__ ko, T* __restrict__ vo, int S,
    int Hq, int Hkv, int hd, int TT, int ks, int flags) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  T* sm = reinterpret_cast<T*>(smem_raw);
  const int L = Hq * hd, K = Hkv * hd, CW = L + K;
  const int hw = ks - 1;               // each causal conv reaches ks-1 tokens back
  T* xs = sm;                          // rows: tokens s0-2hw .. s0+TT-1
  T* y1 = xs + (TT + 2 * hw) * CW;     // rows: tokens s0-hw .. s0+TT-1
  T* y2 = y1 + (TT + hw) * CW;         // rows: tokens s0   .. s0+TT-1
  const int tid = threadIdx.x;
  const int b = blockIdx.y;
  const int s0 = blockIdx.x * TT;
  const bool convs = flags & HYDRA_CCGQA_CONVS;
  const bool qk_mean = flags & HYDRA_CCGQA_QK_MEAN;
  const bool vshift = flags & HYDRA_CCGQA_VALUE_SHIFT;
  const bool qk_norm = flags & HYDRA_CCGQA_QK_NORM;
  const bool rope = flags & HYDRA_CCGQA_ROPE;
  const T* xb = qkv + static_cast<int64_t>(b) * S * qkv_rs;

  for (int i = tid; i < (TT + 2 * hw) * CW; i += 256) {
    const int r = i / CW, c = i - r * CW;
    const int s = s0 - 2 * hw + r;
    xs[i] = (s >= 0 && s < S) ? xb[static_cast<int64_t>(s) * qkv_rs + c] : from_f32<T>(0.f);
  }
  __syncthreads();

  if (convs) {
    // conv1 (grouped): output channel o of group g reads channels g*hd..g*hd+hd-1.
    for (int i = tid; i < (TT + hw) * CW; i += 256) {
      const int r = i / CW, o = i - r * CW;
      const int s = s0 - hw + r;
      float acc = 0.f;
      if (s >= 0 && s < S) {
        const bool is_q = o < L;
        const int oo = is_q ? o : o - L;
        const int col0 = (is_q ? 0 : L) + (oo / hd) * hd;
        const int O = is_q ? L : K;
        for (int t = 0; t < ks; ++t) {
          const T* w = (is_q ? wq1 : wk1) + (static_cast<int64_t>(t) * O + oo) * hd;
          const T* xr = xs + (r + t) * CW + col0;
          for (int c = 0; c < hd; ++c) acc = fmaf(to_f32(w[c]), to_f32(xr[c]), acc);
        }
      }
      y1[i] = from_f32<T>(acc);  // conv2's causal padding is zeros: s < 0 -> 0
    }
    __syncthreads();
    // conv2 (dense over the q or k channels).
    for (int i = tid; i < TT * CW; i += 256) {
      const int r = i / CW, o = i - r * CW;
      const bool is_q = o < L;
      const int oo = is_q ? o : o - L;
      const int C = is_q ? L : K;
      const int col0 = is_q ? 0 : L;
      float acc = 0.f;
      for (int t = 0; t < ks; ++t) {
        const T* w = (is_q ? wq2 : wk2) + (static_cast<int64_t>(t) * C + oo) * C;
        const T* yr = y1 + (r + t) * CW + col0;
        for (int c = 0; c < C; ++c) acc = fmaf(to_f32(w[c]), to_f32(yr[c]), acc);
      }
      y2[i] = from_f32<T>(acc);
    }
  } else {
    for (int i = tid; i < TT * CW; i += 256) y2[i] = xs[2 * hw * CW + i];
  }
  __syncthreads();

  const int G = Hq / Hkv;
  const float tval = (qk_norm && temp) ? to_f32(temp[0]) : 1.f;
  // Epilogue: one thread per (token, head); q heads first, then k heads.
  for (int i = tid; i < TT * (Hq + Hkv); i += 256) {
    const int r = i / (Hq + Hkv), hh = i - r * (Hq + Hkv);
    const int s = s0 + r;
    if (s >= S) continue;
    const bool is_k = hh >= Hq;
    const int head = is_k ? hh - Hq : hh;
    const int col0 = (is_k ? L : 0) + head * hd;
    T* row = y2 + r * CW + col0;
    const T* x0 = xs + (r + 2 * hw) * CW;  // pre-conv q0 | k0 of this token
    if (qk_mean) {
      for (int d = 0; d < hd; ++d) {
        float add;
        if (G == 1) {
          // qk_mean = 0.5 * (q_pre + k_pre), same channel for q and k
          const int c = head * hd + d;
          add = rnd<T>(0.5f * rnd<T>(to_f32(x0[c]) + to_f32(x0[L + c])));
        } else if (is_k) {
          float acc = 0.f;  // mean over query heads of q_pre
          for (int hq = 0; hq < Hq; ++hq) acc += to_f32(x0[hq * hd + d]);
          add = rnd<T>(0.5f * rnd<T>(acc / static_cast<float>(Hq)));
        } else {
          float acc = 0.f;  // mean over kv heads of k_pre
          for (int hk = 0; hk < Hkv; ++hk) acc += to_f32(x0[L + hk * hd + d]);
          add = rnd<T>(0.5f * rnd<T>(acc / static_cast<float>(Hkv)));
        }
        row[d] = from_f32<T>(to_f32(row[d]) + add);
      }
    }
    float fac = 1.f;
    if (qk_norm) {
      float ss = 0.f;
      for (int d = 0; d < hd; ++d) {
        const float f = to_f32(row[d]);
        ss = fmaf(f, f, ss);
      }
      const float nrm = fmaxf(rnd<T>(sqrtf(ss)), 1e-12f);
      fac = nrm;
    }
    T* dst = (is_k ? ko : qo) +
             ((static_cast<int64_t>(b) * (is_k ? Hkv : Hq) + head) * S + s) * hd;
    const float* cr = cs + static_cast<int64_t>(s) * cs_rs;
    const float* sr = sn + static_cast<int64_t>(s) * cs_rs;
    for (int p = 0; p < hd / 2; ++p) {
      float x1 = to_f32(row[2 * p]), x2 = to_f32(row[2 * p + 1]);
      if (qk_norm) {
        x1 = rnd<T>(x1 / fac);
        x2 = rnd<T>(x2 / fac);
        if (is_k) {
          x1 = rnd<T>(x1 * tval);
          x2 = rnd<T>(x2 * tval);
        }
      }
      if (rope) {
        const float c = cr[p], sv = sr[p];
        const float o1 = x1 * c - x2 * sv;
        const float o2 = x1 * sv + x2 * c;
        x1 = o1;
        x2 = o2;
      }
      dst[2 * p] = from_f32<T>(x1);
      dst[2 * p + 1] = from_f32<T>(x2);
    }
  }

  // v with the value shift, written per kv head.
  for (int i = tid; i < TT * K; i += 256) {
    const int r = i / K, c = i - r * K;
    const int s = s0 + r;
    if (s >= S) continue;
    T val;
    if (vshift && c >= K / 2) {
      val = s > 0 ? xb[static_cast<int64_t>(s - 1) * qkv_rs + L + K + c] : from_f32<T>(0.f);
    } else {
      val = xb[static_cast<int64_t>(s) * qkv_rs + L + K + c];
    }
    const int j = c / hd, d = c - j * hd;
    if (flags & HYDRA_CCGQA_V_TRANSPOSED)
      vo[((static_cast<int64_t>(b) * Hkv + j) * hd + d) * S + s] = val;
    else
      vo[((static_cast<int64_t>(b) * Hkv + j) * S + s) * hd + d] = val;
  }
}


// ===========================================================================
// VALU variant for the shapes the MFMA kernel does not take (fp32, fp16,
// odd head layouts): TT = 8 (or 4) tokens per workgroup, fp32 LDS rows.  A thread
// owns one output channel at a time and keeps the tile's TT (conv2) or
// TT + 2 (conv1) token accumulators in registers, so each weight element it
// reads (tap-major rows, 4 consecutive input channels per step) feeds TT
// FMAs, and the token rows come from LDS as 16-byte broadcast reads.
// Rounding points as in ccgqa_prep_generic_kernel.
// ===========================================================================

template <typename T>
__device__ __forceinline__ void ld4(const T* p, float* out) {
  if constexpr (sizeof(T) == 4) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    T a, b2, c, d;
    a.bits = v.x & 0xffffu; b2.bits = v.x >> 16; c.bits = v.y & 0xffffu; d.bits = v.y >> 16;
    out[0] = to_f32(a); out[1] = to_f32(b2); out[2] = to_f32(c); out[3] = to_f32(d);
  }
}

template <typename T, int TT>
__global__ __launch_bounds__(256) void ccgqa_prep_vec_kernel(
    const T* __restrict__ qkv, int64_t qkv_rs, const T* __restrict__ wq1,
    const T* __restrict__ wq2, const T* __restrict__ wk1, const T* __restrict__ wk2,
    const T* __restrict__ temp, const float* __restrict__ cs, const float* __restrict__ sn,
    int64_t cs_rs, T* __restrict__ qo, T* __restrict__ ko, T* __restrict__ vo, int S,
    int Hq, int Hkv, int hd, int flags) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  float* sm = reinterpret_cast<float*>(smem_raw);
  const int L = Hq * hd, K = Hkv * hd, CW = L + K;
  float* xs = sm;                    // rows: tokens s0-4 .. s0+TT-1
  float* y1 = xs + (TT + 4) * CW;    // rows: tokens s0-2 .. s0+TT-1
  float* y2 = y1 + (TT + 2) * CW;    // rows: tokens s0   .. s0+TT-1
  const int tid = threadIdx.x, nth = blockDim.x;
  const int b = blockIdx.y;
  const int s0 = blockIdx.x * TT;
  const bool convs = flags & HYDRA_CCGQA_CONVS;
  const bool qk_mean = flags & HYDRA_CCGQA_QK_MEAN;
  const bool vshift = flags & HYDRA_CCGQA_VALUE_SHIFT;
  const bool qk_norm = flags & HYDRA_CCGQA_QK_NORM;
  const bool rope = flags & HYDRA_CCGQA_ROPE;
  const T* xb = qkv + static_cast<int64_t>(b) * S * qkv_rs;

  for (int i = tid; i < (TT + 4) * CW; i += nth) {
    const int r = i / CW, c = i - r * CW;
    const int s = s0 - 4 + r;
    xs[i] = (s >= 0 && s < S) ? to_f32(xb[static_cast<int64_t>(s) * qkv_rs + c]) : 0.f;
  }
  __syncthreads();

  if (convs) {
    // conv1 (grouped): output o of group g reads channels g*hd .. g*hd+hd-1
    // of rows r .. r+2 (tap t = row offset); outputs of tokens < 0 stay 0
    // (conv2's causal padding).
    for (int o = tid; o < CW; o += nth) {
      const bool is_q = o < L;
      const int oo = is_q ? o : o - L, O = is_q ? L : K;
      const int col0 = (is_q ? 0 : L) + (oo / hd) * hd;
      float acc[TT + 2];
#pragma unroll
      for (int r = 0; r < TT + 2; ++r) acc[r] = 0.f;
      for (int t = 0; t < 3; ++t) {
        const T* w = (is_q ? wq1 : wk1) + (static_cast<int64_t>(t) * O + oo) * hd;
        for (int c = 0; c < hd; c += 4) {
          float wv[4];
          ld4(w + c, wv);
#pragma unroll
          for (int r = 0; r < TT + 2; ++r) {
            const float4 xv = *reinterpret_cast<const float4*>(xs + (r + t) * CW + col0 + c);
            acc[r] = fmaf(wv[0], xv.x, fmaf(wv[1], xv.y, fmaf(wv[2], xv.z, fmaf(wv[3], xv.w, acc[r]))));
          }
        }
      }
#pragma unroll
      for (int r = 0; r < TT + 2; ++r) {
        const int s = s0 - 2 + r;
        y1[r * CW + o] = (s >= 0 && s < S) ? rnd<T>(acc[r]) : 0.f;
      }
    }
    __syncthreads();
    // conv2 (dense over the q or the k channels)
    for (int o = tid; o < CW; o += nth) {
      const bool is_q = o < L;
      const int oo = is_q ? o : o - L, C = is_q ? L : K;
      const int col0 = is_q ? 0 : L;
      float acc[TT];
#pragma unroll
      for (int r = 0; r < TT; ++r) acc[r] = 0.f;
      for (int t = 0; t < 3; ++t) {
        const T* w = (is_q ? wq2 : wk2) + (static_cast<int64_t>(t) * C + oo) * C;
        for (int c = 0; c < C; c += 4) {
          float wv[4];
          ld4(w + c, wv);
#pragma unroll
          for (int r = 0; r < TT; ++r) {
            const float4 yv = *reinterpret_cast<const float4*>(y1 + (r + t) * CW + col0 + c);
            acc[r] = fmaf(wv[0], yv.x, fmaf(wv[1], yv.y, fmaf(wv[2], yv.z, fmaf(wv[3], yv.w, acc[r]))));
          }
        }
      }
#pragma unroll
      for (int r = 0; r < TT; ++r) y2[r * CW + o] = rnd<T>(acc[r]);
    }
  } else {
    for (int i = tid; i < TT * CW; i += nth) y2[i] = xs[4 * CW + i];
  }
  __syncthreads();

  const int G = Hq / Hkv;
  const float tval = (qk_norm && temp) ? to_f32(temp[0]) : 1.f;
  // Epilogue: one thread per (token, head); q heads first, then k heads.
  for (int i = tid; i < TT * (Hq + Hkv); i += nth) {
    const int r = i / (Hq + Hkv), hh = i - r * (Hq + Hkv);
    const int s = s0 + r;
    if (s >= S) continue;
    const bool is_k = hh >= Hq;
    const int head = is_k ? hh - Hq : hh;
    float* row = y2 + r * CW + (is_k ? L : 0) + head * hd;
    const float* x0 = xs + (r + 4) * CW;  // pre-conv q0 | k0 of this token
    if (qk_mean) {
      for (int d = 0; d < hd; ++d) {
        float add;
        if (G == 1) {
          const int c = head * hd + d;
          add = rnd<T>(0.5f * rnd<T>(x0[c] + x0[L + c]));
        } else if (is_k) {
          float acc = 0.f;
          for (int hq = 0; hq < Hq; ++hq) acc += x0[hq * hd + d];
          add = rnd<T>(0.5f * rnd<T>(acc / static_cast<float>(Hq)));
        } else {
          float acc = 0.f;
          for (int hk = 0; hk < Hkv; ++hk) acc += x0[L + hk * hd + d];
          add = rnd<T>(0.5f * rnd<T>(acc / static_cast<float>(Hkv)));
        }
        row[d] = rnd<T>(row[d] + add);
      }
    }
    float fac = 1.f;
    if (qk_norm) {
      float ss = 0.f;
      for (int d = 0; d < hd; ++d) ss = fmaf(row[d], row[d], ss);
      fac = fmaxf(rnd<T>(sqrtf(ss)), 1e-12f);
    }
    T* dst = (is_k ? ko : qo) + ((static_cast<int64_t>(b) * (is_k ? Hkv : Hq) + head) * S + s) * hd;
    const float* cr = cs + static_cast<int64_t>(s) * cs_rs;
    const float* sr = sn + static_cast<int64_t>(s) * cs_rs;
    for (int pp = 0; pp < hd / 2; ++pp) {
      float x1 = row[2 * pp], x2 = row[2 * pp + 1];
      if (qk_norm) {
        x1 = rnd<T>(x1 / fac);
        x2 = rnd<T>(x2 / fac);
        if (is_k) {
          x1 = rnd<T>(x1 * tval);
          x2 = rnd<T>(x2 * tval);
        }
      }
      if (rope) {
        const float c = cr[pp], sv = sr[pp];
        const float o1 = x1 * c - x2 * sv;
        const float o2 = x1 * sv + x2 * c;
        x1 = o1;
        x2 = o2;
      }
      dst[2 * pp] = from_f32<T>(x1);
      dst[2 * pp + 1] = from_f32<T>(x2);
    }
  }

  // v with the value shift, written per kv head.
  for (int i = tid; i < TT * K; i += nth) {
    const int r = i / K, c = i - r * K;
    const int s = s0 + r;
    if (s >= S) continue;
    T val;
    if (vshift && c >= K / 2) {
      val = s > 0 ? xb[static_cast<int64_t>(s - 1) * qkv_rs + L + K + c] : from_f32<T>(0.f);
    } else {
      val = xb[static_cast<int64_t>(s) * qkv_rs + L + K + c];
    }
    const int j = c / hd, d = c - j * hd;
    if (flags & HYDRA_CCGQA_V_TRANSPOSED)
      vo[((static_cast<int64_t>(b) * Hkv + j) * hd + d) * S + s] = val;
    else
      vo[((static_cast<int64_t>(b) * Hkv + j) * S + s) * hd + d] = val;
  }
}

// ===========================================================================
// bf16 MFMA variant.
//
// LDS (bf16, rows padded by 8 elements): X = qkv q|k columns of tokens
// [s0-4, s0+TT), Y1 = conv1 output of tokens [s0-2, s0+TT), and the RoPE
// cos/sin rows of the tile (fp32).  Both convs are computed transposed,
//   Y^T[o, s] = sum_t sum_c W[t][o][c] * In[s + t - 2, c],
// as 32(out channels) x 32(tokens) MFMA tiles: A = weights straight from
// global (L2-resident, 16-byte loads along c, a ring of loads in flight),
// B = token rows from LDS (16 bytes along c), so lane l owns token l%32.
// A task is one 32-channel m-tile times every token tile (conv1: of the
// TT+2 rows conv2 needs), so each weight fragment is read once per
// workgroup and feeds TT/32 (+1) MFMAs; the tasks of both convs are spread
// over all 8 waves.  conv2's output, rounded to bf16, goes to LDS, and the
// epilogue (QK-mean, L2-norm with temperature, RoPE) runs on all threads
// with 8 channels per lane.
// ===========================================================================
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_p;
typedef __attribute__((ext_vector_type(16))) float f32x16_p;

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_p;

__device__ __forceinline__ bf16x8_p ld_bf16x8(const void* p) {
  return __builtin_bit_cast(bf16x8_p, *reinterpret_cast<const uint4*>(p));
}

// acc + a.lo*b.lo + a.hi*b.hi on packed bf16 pairs (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_p, a),
                                         __builtin_bit_cast(bf16x2_p, b), acc, false);
}

// One MFMA conv task: the 32 output channels of the m-tile (weight rows
// from wbase, lane row n, k half hf) times all NT token tiles, over 3 taps x
// CS k-steps of 16 input channels.  A (weights) streams from L2, B (token
// rows) from LDS at bbase + brow(j, t).  With CS known at compile time the
// 3*CS steps are unrolled and the A fragments run through a ring of D
// registers, so D L2 loads stay in flight behind the MFMAs; otherwise a
// plain loop.
template <int CS>
struct ConvRing {
  static constexpr int NSTEP = 3 * CS;
  static constexpr int D = NSTEP < 12 ? NSTEP : 12;  // A steps in flight
};

// The first ConvRing<CS>::D A fragments of a conv task (see below), issued
// ahead of the task (e.g. before the barrier that ends the staging).
template <int CS>
__device__ __forceinline__ void conv_ring_fill(const bf16* wbase, int64_t wtap, int wstep,
                                               bf16x8_p (&ring)[ConvRing<CS>::D]) {
#pragma unroll
  for (int i = 0; i < ConvRing<CS>::D; ++i) ring[i] = ld_bf16x8(wbase + (i / CS) * wtap + wstep * (i % CS));
}

template <int NT, int CS, typename BRow>
__device__ __forceinline__ void conv_task_fixed(const bf16* wbase, int64_t wtap, int wstep,
                                                const uint16_t* bbase, BRow brow,
                                                f32x16_p (&acc)[NT],
                                                const bf16x8_p* pre = nullptr) {
  constexpr int NSTEP = ConvRing<CS>::NSTEP;
  constexpr int D = ConvRing<CS>::D;  // A steps in flight
  bf16x8_p ring[D];
  bf16x8_p bq[2][NT];  // B fragments of this step and the next
  auto aptr = [&](int st) { return wbase + (st / CS) * wtap + wstep * (st % CS); };
  auto bload = [&](int st, bf16x8_p* dst) {
#pragma unroll
    for (int j = 0; j < NT; ++j) dst[j] = ld_bf16x8(bbase + brow(j, st / CS) + 16 * (st % CS));
  };
#pragma unroll
  for (int i = 0; i < D; ++i) ring[i] = pre ? pre[i] : ld_bf16x8(aptr(i));
  bload(0, bq[0]);
#pragma unroll
  for (int st = 0; st < NSTEP; ++st) {
    const bf16x8_p a = ring[st % D];
    if (st + 1 < NSTEP) bload(st + 1, bq[(st + 1) & 1]);
    if (st + D < NSTEP) ring[st % D] = ld_bf16x8(aptr(st + D));
    // Keep the scheduler from sinking the loads next to their use: they
    // hide L2 and LDS latency only if they really are in flight.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NT; ++j)
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bq[st & 1][j], acc[j], 0, 0, 0);
  }
}

template <int NT, typename BRow>
__device__ __forceinline__ void conv_task(const bf16* wbase, int64_t wtap, int wstep, int CS,
                                          const uint16_t* bbase, BRow brow,
                                          f32x16_p (&acc)[NT]) {
  switch (CS) {  // CS is uniform: a scalar branch
    case 1: return conv_task_fixed<NT, 1>(wbase, wtap, wstep, bbase, brow, acc);
    case 2: return conv_task_fixed<NT, 2>(wbase, wtap, wstep, bbase, brow, acc);
    case 4: return conv_task_fixed<NT, 4>(wbase, wtap, wstep, bbase, brow, acc);
    case 8: return conv_task_fixed<NT, 8>(wbase, wtap, wstep, bbase, brow, acc);
    default: break;
  }
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    const bf16* wt = wbase + t * wtap;
    const uint16_t* bt[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) bt[j] = bbase + brow(j, t);
#pragma unroll 8
    for (int c = 0; c < CS; ++c) {
      const bf16x8_p a = ld_bf16x8(wt + wstep * c);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const bf16x8_p bb = ld_bf16x8(bt[j] + 16 * c);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, bb, acc[j], 0, 0, 0);
      }
    }
  }
}

// conv1 of an m-tile when head_dim is 16: its 32 output channels are two
// groups of 16 with different inputs (channels cbase..cbase+15 for rows
// 0..15, cbase+16..cbase+31 for rows 16..31), i.e. a block-diagonal 32 x 32
// weight.  Each tap runs two k-steps over the 32 inputs with the A fragment
// (lane row n, which the weight layout gives as W[o0+n][8 hf .. 8 hf + 8])
// zeroed in the step of the other group.
template <int NT, typename BRow>
__device__ __forceinline__ void conv1_task_hd16(const bf16* wbase, int64_t wtap,
                                                const uint16_t* bbase, BRow brow, int n,
                                                f32x16_p (&acc)[NT]) {
  const bf16x8_p zero = {};
  bf16x8_p a[3];
#pragma unroll
  for (int t = 0; t < 3; ++t) a[t] = ld_bf16x8(wbase + t * wtap);
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    const bf16x8_p a0 = n < 16 ? a[t] : zero, a1 = n < 16 ? zero : a[t];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const bf16x8_p b0 = ld_bf16x8(bbase + brow(j, t));
      const bf16x8_p b1 = ld_bf16x8(bbase + brow(j, t) + 16);
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[j], 0, 0, 0);
      acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[j], 0, 0, 0);
    }
  }
}

// One conv2 task: the MT m-tiles (32 output channels each) of one head times
// NG 32-token tiles.  Each step's MT A fragments (weights) and NG B fragments
// (token rows from LDS, row 32g + n + t for tap t) feed MT x NG MFMAs; A runs
// through a ring of D steps of loads in flight, B one step ahead.
template <int MT, int NG, int CS>
__device__ __forceinline__ void conv2_task_fixed(const bf16* wrow, int64_t wtap, int64_t wmt,
                                                 int wstep, const uint16_t* brow0, int rs,
                                                 f32x16_p (&acc)[MT][NG]) {
  constexpr int NSTEP = 3 * CS;
  constexpr int DW = (MT * NG >= 8 ? 8 : 16) / MT;  // A steps in flight
  constexpr int D = NSTEP < DW ? NSTEP : (DW > 0 ? DW : 1);
  bf16x8_p ring[D][MT];
  bf16x8_p bq[2][NG];
  auto aptr = [&](int st, int m) { return wrow + (st / CS) * wtap + m * wmt + wstep * (st % CS); };
  auto bload = [&](int st, bf16x8_p* dst) {
#pragma unroll
    for (int g = 0; g < NG; ++g) dst[g] = ld_bf16x8(brow0 + (32 * g + st / CS) * rs + 16 * (st % CS));
  };
#pragma unroll
  for (int i = 0; i < D; ++i)
#pragma unroll
    for (int m = 0; m < MT; ++m) ring[i][m] = ld_bf16x8(aptr(i, m));
  bload(0, bq[0]);
#pragma unroll
  for (int st = 0; st < NSTEP; ++st) {
    bf16x8_p a[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) a[m] = ring[st % D][m];
    if (st + 1 < NSTEP) bload(st + 1, bq[(st + 1) & 1]);
#pragma unroll
    for (int m = 0; m < MT; ++m)
      if (st + D < NSTEP) ring[st % D][m] = ld_bf16x8(aptr(st + D, m));
    // Keep the scheduler from sinking the loads next to their use: they
    // hide L2 and LDS latency only if they really are in flight.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
      for (int g = 0; g < NG; ++g)
        acc[m][g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[m], bq[st & 1][g], acc[m][g], 0, 0, 0);
  }
}

template <int MT, int NG>
__device__ __forceinline__ void conv2_task(const bf16* wrow, int64_t wtap, int64_t wmt, int wstep,
                                           int CS, const uint16_t* brow0, int rs,
                                           f32x16_p (&acc)[MT][NG]) {
  switch (CS) {  // uniform
    case 2: return conv2_task_fixed<MT, NG, 2>(wrow, wtap, wmt, wstep, brow0, rs, acc);
    case 4: return conv2_task_fixed<MT, NG, 4>(wrow, wtap, wmt, wstep, brow0, rs, acc);
    case 8: return conv2_task_fixed<MT, NG, 8>(wrow, wtap, wmt, wstep, brow0, rs, acc);
    case 16: return conv2_task_fixed<MT, NG, 16>(wrow, wtap, wmt, wstep, brow0, rs, acc);
    default: break;
  }
  if constexpr (MT == 1) {
    // head_dim <= 32 (one m-tile per task): the latent widths 192, 320,
    // 384, 448 (the 1B preset: 28 heads of 16) and 512 get the pipelined
    // weight stream too (at MT > 1 the longer unrolled bodies would spill)
    switch (CS) {
      case 12: return conv2_task_fixed<MT, NG, 12>(wrow, wtap, wmt, wstep, brow0, rs, acc);
      case 20: return conv2_task_fixed<MT, NG, 20>(wrow, wtap, wmt, wstep, brow0, rs, acc);
      case 24: return conv2_task_fixed<MT, NG, 24>(wrow, wtap, wmt, wstep, brow0, rs, acc);
      case 28: return conv2_task_fixed<MT, NG, 28>(wrow, wtap, wmt, wstep, brow0, rs, acc);
      case 32: return conv2_task_fixed<MT, NG, 32>(wrow, wtap, wmt, wstep, brow0, rs, acc);
      default: break;
    }
  }
  for (int t = 0; t < 3; ++t)
    for (int c = 0; c < CS; ++c) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const bf16x8_p bb = ld_bf16x8(brow0 + (32 * g + t) * rs + 16 * c);
#pragma unroll
        for (int m = 0; m < MT; ++m)
          acc[m][g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              ld_bf16x8(wrow + t * wtap + m * wmt + wstep * c), bb, acc[m][g], 0, 0, 0);
      }
    }
}

// 8 waves: two per SIMD, so one wave's VALU work and L2 latency overlap
// another's MFMAs.
constexpr int kPrepThreads = 512;

template <int HD, int TT>
__global__ __launch_bounds__(kPrepThreads) void ccgqa_prep_mfma_kernel(
    const bf16* __restrict__ qkv, int64_t qkv_rs, const bf16* __restrict__ wq1,
    const bf16* __restrict__ wq2, const bf16* __restrict__ wk1, const bf16* __restrict__ wk2,
    const bf16* __restrict__ temp, const float* __restrict__ cs, const float* __restrict__ sn,
    int64_t cs_rs, bf16* __restrict__ qo, bf16* __restrict__ ko, bf16* __restrict__ vo, int S,
    int Hq, int Hkv, int flags) {
  constexpr int NT = TT / 32;  // token tiles
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  uint16_t* sm = reinterpret_cast<uint16_t*>(smem_raw);
  const int L = Hq * HD, K = Hkv * HD, CW = L + K, RS = CW + 8;
  const int G = Hq / Hkv;
  // QK-mean terms per token: one per head when G == 1 ((q0_h + k0_h) / 2),
  // else one for the q heads (mean of the k heads) and one for the k heads.
  const int NQA = G == 1 ? Hq : 2;
  uint16_t* X = sm;                   // row r <-> token s0 - 4 + r
  uint16_t* Y1 = X + (TT + 4) * RS;   // row r <-> token s0 - 2 + r
  // RoPE cos | sin of the tile's tokens, fp32 [TT][CSR] each; rows padded
  // by 2 floats so the 32 tokens of a half-wave read distinct banks.
  constexpr int CSR = HD / 2 + 2;
  float* CSl = reinterpret_cast<float*>(Y1 + (TT + 2) * RS);
  float* SNl = CSl + TT * CSR;
  uint16_t* QA = reinterpret_cast<uint16_t*>(SNl + TT * CSR);  // bf16 [TT][QAS]
  // v columns of tokens [s0-1, s0+TT), row r <-> token s0 - 1 + r (the
  // value shift reads the previous token), rows padded by 8 elements
  const int VR = K + 8;
  // QK-mean term rows padded by 8 elements: with NQA*HD a multiple of 64
  // the epilogue's reads of 32 consecutive tokens would share one bank.
  const int QAS = NQA * HD + 8;
  uint16_t* Vs = QA + TT * QAS;
  // count of waves done with the QK-mean terms (see the conv2 phase)
  int* qa_done = reinterpret_cast<int*>(Vs + ((TT + 1) * VR + 7) / 8 * 8);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int n = lane & 31, hf = lane >> 5;
  const int b = blockIdx.y;
  const int s0 = blockIdx.x * TT;
  const bool convs = flags & HYDRA_CCGQA_CONVS;
  const bool qk_mean = flags & HYDRA_CCGQA_QK_MEAN;
  const bool vshift = flags & HYDRA_CCGQA_VALUE_SHIFT;
  const bool qk_norm = flags & HYDRA_CCGQA_QK_NORM;
  const bool rope = flags & HYDRA_CCGQA_ROPE;
  // Weight layout: tap-major rows ([3][O][I], a fragment is 32 rows x 32
  // bytes) or MFMA-tiled ([3][O/32][I/16][64 lanes][8], a fragment is one
  // contiguous 1 KB block).  Both have tap stride O*I and m-tile stride 32*I.
  const bool tiled = flags & HYDRA_CCGQA_W_TILED;
  const int wstep = tiled ? 512 : 16;  // elements between k-steps
  const bf16* xb = qkv + static_cast<int64_t>(b) * S * qkv_rs;

  // conv1 m-tile mt (32 output channels): its weight rows and input columns
  const int nm1 = CW / 32;
  auto conv1_w = [&](int mt) {
    const int o0 = 32 * mt;
    const bool is_q = o0 < L;
    const int oo0 = is_q ? o0 : o0 - L;
    return (is_q ? wq1 : wk1) + static_cast<int64_t>(oo0) * HD + (tiled ? 8 * lane : n * HD + 8 * hf);
  };
  auto conv1_wtap = [&](int mt) { return static_cast<int64_t>(32 * mt < L ? L : K) * HD; };
  // The first m-tile's weight fragments go out before the staging, so
  // their L2 latency overlaps the staging's HBM reads.
  constexpr int CS1 = HD / 16;
  bf16x8_p ring1[ConvRing<CS1>::D];
  const bool pre1 = convs && HD != 16 && wave < nm1;
  if (pre1) conv_ring_fill<CS1>(conv1_w(wave), conv1_wtap(wave), wstep, ring1);

  // ---- stage q0|k0 rows, v rows, RoPE angles --------------------------------
  if (tid == 0) *qa_done = 0;
  // Each round issues all of a thread's 16-byte global loads of the three
  // regions (up to 8 + 2 + 2) before it writes any of them to LDS, so the
  // whole tile is in flight at once; (row, chunk) advance incrementally, with
  // no division per item.
  {
    constexpr int KX = 8, KV = 2, KC = 2;
    constexpr int Q4 = HD / 8;  // float4 chunks per cos (or sin) row
    const int cw8 = CW / 8, k8 = K / 8;
    const int nx = (TT + 4) * cw8, nv = (TT + 1) * k8, nc = rope ? 2 * TT * Q4 : 0;
    const int xq = kPrepThreads / cw8, xm = kPrepThreads - xq * cw8;
    const int vq = kPrepThreads / k8, vm = kPrepThreads - vq * k8;
    int xr = tid / cw8, xc = tid - xr * cw8;
    int vr = tid / k8, vc = tid - vr * k8;
    for (int round = 0;; ++round) {
      const int bx = round * KX * kPrepThreads, bv = round * KV * kPrepThreads,
                bc = round * KC * kPrepThreads;
      if (bx >= nx && bv >= nv && bc >= nc) break;
      uint4 xval[KX], vval[KV], cval[KC];
      int xrr[KX], xcc[KX], vrr[KV], vcc[KV];
#pragma unroll
      for (int j = 0; j < KX; ++j) {
        xrr[j] = xr;
        xcc[j] = xc;
        const int s = s0 - 4 + xr;
        xval[j] = make_uint4(0, 0, 0, 0);
        if (bx + j * kPrepThreads + tid < nx && s >= 0 && s < S)
          xval[j] = *reinterpret_cast<const uint4*>(xb + static_cast<int64_t>(s) * qkv_rs + 8 * xc);
        xr += xq;
        xc += xm;
        if (xc >= cw8) { xc -= cw8; ++xr; }
      }
#pragma unroll
      for (int j = 0; j < KV; ++j) {
        vrr[j] = vr;
        vcc[j] = vc;
        const int s = s0 - 1 + vr;
        vval[j] = make_uint4(0, 0, 0, 0);
        if (bv + j * kPrepThreads + tid < nv && s >= 0 && s < S)
          vval[j] = *reinterpret_cast<const uint4*>(xb + static_cast<int64_t>(s) * qkv_rs + L + K + 8 * vc);
        vr += vq;
        vc += vm;
        if (vc >= k8) { vc -= k8; ++vr; }
      }
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        const int i = bc + j * kPrepThreads + tid;
        const int which = i / (TT * Q4), rem = i - which * (TT * Q4);
        const int r = rem / Q4, c4 = (rem - r * Q4) * 4;
        const int s = s0 + r;
        cval[j] = make_uint4(0, 0, 0, 0);
        if (i < nc && s < S)
          cval[j] = *reinterpret_cast<const uint4*>((which ? sn : cs) + static_cast<int64_t>(s) * cs_rs + c4);
      }
#pragma unroll
      for (int j = 0; j < KX; ++j)
        if (bx + j * kPrepThreads + tid < nx)
          *reinterpret_cast<uint4*>(X + xrr[j] * RS + 8 * xcc[j]) = xval[j];
#pragma unroll
      for (int j = 0; j < KV; ++j)
        if (bv + j * kPrepThreads + tid < nv)
          *reinterpret_cast<uint4*>(Vs + vrr[j] * VR + 8 * vcc[j]) = vval[j];
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        const int i = bc + j * kPrepThreads + tid;
        if (i < nc) {
          const int which = i / (TT * Q4), rem = i - which * (TT * Q4);
          const int r = rem / Q4, c4 = (rem - r * Q4) * 4;
          float* d = (which ? SNl : CSl) + r * CSR + c4;  // 8-byte aligned rows
          *reinterpret_cast<uint2*>(d) = make_uint2(cval[j].x, cval[j].y);
          *reinterpret_cast<uint2*>(d + 2) = make_uint2(cval[j].z, cval[j].w);
        }
      }
    }
  }
  __syncthreads();

  // ---- side work: QK-mean terms into QA ---------------------------------------
  // Shared by the waves [hw0, 8); they run it while the others still have
  // MFMA tasks, so it stays off the critical path.
  auto qa_work = [&](int hw0) {
    if (!qk_mean) return;
    const int hl = (wave - hw0) * 64 + lane, nhl = (kPrepThreads / 64 - hw0) * 64;
    constexpr int C8 = HD / 8;
    const float inv_q = 1.f / static_cast<float>(Hq), inv_k = 1.f / static_cast<float>(Hkv);
    // items ordered [term q][token r][chunk c8]: a wave's lanes share q, so
    // the head loop below does not diverge
    for (int it = hl; it < TT * NQA * C8; it += nhl) {
      const int q = it / (TT * C8), rem = it - q * (TT * C8);
      const int r = rem / C8, c8 = (rem - r * C8) * 8;
      const bf16* x0 = reinterpret_cast<const bf16*>(X + (r + 4) * RS);
      float sum[8];
      float scale;
      if (G == 1) {
        // (q0_h + k0_h) / 2
        float c[8];
        load16<bf16>(x0 + q * HD + c8, sum);
        load16<bf16>(x0 + L + q * HD + c8, c);
#pragma unroll
        for (int e = 0; e < 8; ++e) sum[e] += c[e];
        scale = 1.f;
      } else {
        // term 0 (for q heads): mean of the k heads; term 1: of the q heads
        const int nh = q ? Hq : Hkv;
        const bf16* src = x0 + (q ? 0 : L) + c8;
        load16<bf16>(src, sum);
#pragma unroll 4
        for (int hx = 1; hx < nh; ++hx) {
          float a[8];
          load16<bf16>(src + hx * HD, a);
#pragma unroll
          for (int e = 0; e < 8; ++e) sum[e] += a[e];
        }
        scale = q ? inv_q : inv_k;
      }
      // rnd(0.5 * rnd(mean)), two values per conversion
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const uint32_t m = pack2<bf16>(sum[e] * scale, sum[e + 1] * scale);
        w[e / 2] = pack2<bf16>(0.5f * __uint_as_float(m << 16), 0.5f * __uint_as_float(m & 0xffff0000u));
      }
      *reinterpret_cast<uint4*>(QA + r * QAS + q * HD + c8) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  };
  // v from the staged rows to global: channels of the second half take the
  // previous token with the value shift (row r of token s, row r+1
  // otherwise).  Shared by the waves [hw0, 8).
  auto v_work = [&](int hw0) {
    const int hl = (wave - hw0) * 64 + lane, nhl = (kPrepThreads / 64 - hw0) * 64;
    if (flags & HYDRA_CCGQA_V_TRANSPOSED) {
      // v^T [B, Hkv, hd, S]: 8 consecutive tokens of one channel per
      // 16-byte store
      for (int i = hl; i < K * (TT / 8); i += nhl) {
        const int c = i / (TT / 8), t8 = (i - c * (TT / 8)) * 8;
        const int dr = (vshift && c >= K / 2) ? 0 : 1;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = static_cast<uint32_t>(Vs[(t8 + 2 * e + dr) * VR + c]) |
                 (static_cast<uint32_t>(Vs[(t8 + 2 * e + 1 + dr) * VR + c]) << 16);
        if (s0 + t8 < S) {
          const int j = c / HD, d = c - j * HD;
          *reinterpret_cast<uint4*>(vo + ((static_cast<int64_t>(b) * Hkv + j) * HD + d) * S + s0 + t8) =
              make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
    } else {
      const int k8 = K / 8;
      for (int i = hl; i < TT * k8; i += nhl) {
        const int r = i / k8, c = (i - r * k8) * 8;
        const int s = s0 + r;
        if (s >= S) continue;
        const int dr = (vshift && c >= K / 2) ? 0 : 1;
        const uint4 val = *reinterpret_cast<const uint4*>(Vs + (r + dr) * VR + c);
        const int j = c / HD, d = c - j * HD;
        *reinterpret_cast<uint4*>(vo + ((static_cast<int64_t>(b) * Hkv + j) * S + s) * HD + d) = val;
      }
    }
  };
  const float tval = (qk_norm && temp) ? to_f32(temp[0]) : 1.f;

  if (!convs) {
    // ---- no convs: QK-mean terms and v, then the row epilogue over X --------
    qa_work(0);
    v_work(0);
    __syncthreads();
    // HD/8 lanes per (token, head) row, 8 channels each; a wave covers 8
    // rows, i.e. the heads of consecutive tokens, so RoPE angles are shared
    // reads and every row leaves as one contiguous 2*HD-byte store.
    // Roundings follow the reference: the QK-mean sum, the norm, the
    // normalised vector, the temperature product.
    uint16_t* Y2 = X + 4 * RS;  // row r <-> token s0 + r
    constexpr int LPR = HD / 8;
    const int nheads = Hq + Hkv;
    const int rows = TT * nheads;
    for (int base = 0; base < rows * LPR; base += kPrepThreads) {
      const int i = base + tid;
      const bool live = i < rows * LPR;
      const int row = live ? i / LPR : 0, c8 = (i % LPR) * 8;
      const int r = row / nheads, hh = row - r * nheads;
      const int s = s0 + r;
      const bool is_k = hh >= Hq;
      const int head = is_k ? hh - Hq : hh;
      float v[8];
      load16<bf16>(reinterpret_cast<const bf16*>(Y2 + r * RS + (is_k ? L : 0) + head * HD + c8), v);
      if (qk_mean) {
        float add[8];
        const int q = G == 1 ? head : (is_k ? 1 : 0);
        load16<bf16>(reinterpret_cast<const bf16*>(QA + r * QAS + q * HD + c8), add);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] += add[e];
        rnd8(v);
      }
      if (qk_norm) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
        ss = wave_sum<LPR>(ss);
        const float rinv = 1.f / fmaxf(rnd<bf16>(__builtin_sqrtf(ss)), 1e-12f);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] *= rinv;
        rnd8(v);
        if (is_k) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] *= tval;
          rnd8(v);
        }
      }
      if (rope) {
        const float* cr = CSl + r * CSR + c8 / 2;
        const float* sr = SNl + r * CSR + c8 / 2;
#pragma unroll
        for (int p2 = 0; p2 < 2; ++p2) {
          const float2 cv = *reinterpret_cast<const float2*>(cr + 2 * p2);
          const float2 sv = *reinterpret_cast<const float2*>(sr + 2 * p2);
          const float x0 = v[4 * p2 + 0], x1 = v[4 * p2 + 1], x2 = v[4 * p2 + 2], x3 = v[4 * p2 + 3];
          v[4 * p2 + 0] = x0 * cv.x - x1 * sv.x;
          v[4 * p2 + 1] = x0 * sv.x + x1 * cv.x;
          v[4 * p2 + 2] = x2 * cv.y - x3 * sv.y;
          v[4 * p2 + 3] = x2 * sv.y + x3 * cv.y;
        }
      }
      if (live && s < S) {
        bf16* dst = (is_k ? ko : qo) +
                    ((static_cast<int64_t>(b) * (is_k ? Hkv : Hq) + head) * S + s) * HD + c8;
        store16<bf16>(dst, v);
      }
    }
    return;
  }

  // ---- conv1 on MFMA ----------------------------------------------------------
  // Output row i in [0, TT+2) <-> token s0-2+i reads X rows i..i+2.  The
  // rows are covered by NT+1 token tiles; the last holds the two rows past
  // TT (its other lanes read clamped rows and are discarded).  Rows of
  // tokens < 0 come out 0 (their X rows are 0): conv2's causal padding.
  {
    constexpr int NT1 = NT + 1;
    for (int mt = wave; mt < nm1; mt += kPrepThreads / 64) {
      const int o0 = 32 * mt;
      const bool is_q = o0 < L;
      const int oo0 = is_q ? o0 : o0 - L;
      const int cbase = (is_q ? 0 : L) + (oo0 / HD) * HD;
      const bf16* wbase = conv1_w(mt);
      f32x16_p acc[NT1];
#pragma unroll
      for (int j = 0; j < NT1; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
      auto brow1 = [&](int j, int t) { return min(32 * j + n + t, TT + 3) * RS; };
      if constexpr (HD == 16)
        conv1_task_hd16<NT1>(wbase, conv1_wtap(mt), X + cbase + 8 * hf, brow1, n, acc);
      else if (mt == wave)  // the prefetched first m-tile
        conv_task_fixed<NT1, CS1>(wbase, conv1_wtap(mt), wstep, X + cbase + 8 * hf, brow1, acc, ring1);
      else
        conv_task<NT1>(wbase, conv1_wtap(mt), wstep, HD / 16, X + cbase + 8 * hf, brow1, acc);
#pragma unroll
      for (int j = 0; j < NT1; ++j) {
        const int i = 32 * j + n;
        if (j < NT || i < TT + 2) {
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            uint2 w;
            w.x = pack2<bf16>(acc[j][4 * g4 + 0], acc[j][4 * g4 + 1]);
            w.y = pack2<bf16>(acc[j][4 * g4 + 2], acc[j][4 * g4 + 3]);
            *reinterpret_cast<uint2*>(Y1 + i * RS + o0 + 8 * g4 + 4 * hf) = w;
          }
        }
      }
    }
    // With at least one conv2 task per wave, the waves with one conv1
    // m-tile fewer compute the QK-mean terms here; otherwise the waves
    // without a conv2 task do it during conv2.
    const int HPT2 = HD >= 32 ? 1 : 32 / HD;
    const int extra = nm1 % (kPrepThreads / 64);
    if ((Hq + Hkv) / HPT2 >= kPrepThreads / 64 && wave >= extra) qa_work(extra);
  }
  __syncthreads();

  // ---- conv2 on MFMA with the epilogue on its accumulators ---------------------
  // A task is 32 * MT output channels (one head when HD >= 32, one 32-channel
  // m-tile of two heads when HD = 16) times all NT token tiles, so each
  // weight fragment is read once per workgroup.  Output token s0+32j+n, tap
  // t reads Y1 row 32j+n+t.  In the 32x32 MFMA result lane (n, hf) holds
  // token 32j+n, channels 32m + 8*g4 + 4*hf + e (e < 4): the epilogue
  // (rounding of the conv output, QK-mean term, L2 norm with the partner
  // lane's half (lane ^ 32), temperature, RoPE on the (e0,e1), (e2,e3)
  // pairs) runs in registers, and channel groups are regrouped across the
  // half-waves (v_permlane32_swap) so each lane writes 16 contiguous bytes.
  // When there are fewer tasks than waves, the waves without one compute the
  // QK-mean terms meanwhile (one barrier before the epilogues) and then v.
  {
    constexpr int MT = HD >= 32 ? HD / 32 : 1;
    constexpr int HPT = HD >= 32 ? 1 : 32 / HD;  // heads per task
    constexpr int NHL = HD >= 32 ? 1 : 2;         // heads in a lane's channels
    constexpr int NW = kPrepThreads / 64;
    const int ntask = (Hq + Hkv) / HPT;
    auto mfma = [&](int task, f32x16_p (&acc)[MT][NT]) {
      const int hh = task * HPT;
      const bool is_k = hh >= Hq;
      const int head0 = is_k ? hh - Hq : hh;
      const int C = is_k ? K : L;
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[m][j][r] = 0.f;
      conv2_task<MT, NT>((is_k ? wk2 : wq2) + static_cast<int64_t>(head0 * HD) * C +
                             (tiled ? 8 * lane : n * C + 8 * hf),
                         static_cast<int64_t>(C) * C, static_cast<int64_t>(32) * C, wstep, C / 16,
                         Y1 + n * RS + (is_k ? L : 0) + 8 * hf, RS, acc);
    };
    auto epilogue = [&](int task, f32x16_p (&acc)[MT][NT]) {
      const int hh = task * HPT;
      const bool is_k = hh >= Hq;
      const int head0 = is_k ? hh - Hq : hh;
      const int Hn = is_k ? Hkv : Hq;
      const int q0 = G == 1 ? head0 : (is_k ? 1 : 0);  // QK-mean term row
      bf16* obase = (is_k ? ko : qo) + ((static_cast<int64_t>(b) * Hn + head0) * S + s0) * HD;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int t = 32 * j + n;
        // conv output rounded to bf16 (the reference materialises it)
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int i = 0; i < 16; i += 2) {
            const uint32_t p = pack2<bf16>(acc[m][j][i], acc[m][j][i + 1]);
            acc[m][j][i] = __uint_as_float(p << 16);
            acc[m][j][i + 1] = __uint_as_float(p & 0xffff0000u);
          }
        if (qk_mean) {
          const uint16_t* qa = QA + t * QAS + q0 * HD + 4 * hf;
#pragma unroll
          for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              const int tc = 32 * m + 8 * g4;
              const int off = (G == 1 ? (tc / HD) * HD : 0) + tc % HD;
              const uint2 w = *reinterpret_cast<const uint2*>(qa + off);
              f32x16_p& a = acc[m][j];
              const uint32_t p0 = pack2<bf16>(a[4 * g4 + 0] + __uint_as_float(w.x << 16),
                                              a[4 * g4 + 1] + __uint_as_float(w.x & 0xffff0000u));
              const uint32_t p1 = pack2<bf16>(a[4 * g4 + 2] + __uint_as_float(w.y << 16),
                                              a[4 * g4 + 3] + __uint_as_float(w.y & 0xffff0000u));
              a[4 * g4 + 0] = __uint_as_float(p0 << 16);
              a[4 * g4 + 1] = __uint_as_float(p0 & 0xffff0000u);
              a[4 * g4 + 2] = __uint_as_float(p1 << 16);
              a[4 * g4 + 3] = __uint_as_float(p1 & 0xffff0000u);
            }
        }
        if (qk_norm) {
          float ss[NHL];
#pragma unroll
          for (int h = 0; h < NHL; ++h) ss[h] = 0.f;
#pragma unroll
          for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int h = NHL == 1 ? 0 : (i / 4) / 2;
              ss[h] = fmaf(acc[m][j][i], acc[m][j][i], ss[h]);
            }
          float rinv[NHL];
#pragma unroll
          for (int h = 0; h < NHL; ++h)
            rinv[h] = 1.f / fmaxf(rnd<bf16>(__builtin_sqrtf(halves_sum(ss[h]))), 1e-12f);
#pragma unroll
          for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int i = 0; i < 16; i += 2) {
              const int h = NHL == 1 ? 0 : (i / 4) / 2;
              uint32_t p = pack2<bf16>(acc[m][j][i] * rinv[h], acc[m][j][i + 1] * rinv[h]);
              if (is_k)
                p = pack2<bf16>(__uint_as_float(p << 16) * tval, __uint_as_float(p & 0xffff0000u) * tval);
              acc[m][j][i] = __uint_as_float(p << 16);
              acc[m][j][i + 1] = __uint_as_float(p & 0xffff0000u);
            }
        }
        if (rope) {
          const float* cr = CSl + t * CSR + 2 * hf;
          const float* sr = SNl + t * CSR + 2 * hf;
#pragma unroll
          for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              const int off = ((32 * m + 8 * g4) % HD) / 2;
              const float2 cv = *reinterpret_cast<const float2*>(cr + off);
              const float2 sv = *reinterpret_cast<const float2*>(sr + off);
              f32x16_p& a = acc[m][j];
              const float x0 = a[4 * g4 + 0], x1 = a[4 * g4 + 1];
              const float x2 = a[4 * g4 + 2], x3 = a[4 * g4 + 3];
              a[4 * g4 + 0] = x0 * cv.x - x1 * sv.x;
              a[4 * g4 + 1] = x0 * sv.x + x1 * cv.x;
              a[4 * g4 + 2] = x2 * cv.y - x3 * sv.y;
              a[4 * g4 + 3] = x2 * sv.y + x3 * cv.y;
            }
        }
        // groups g4 = 2p and 2p+1 swap halves: lane hf ends with the 8
        // channels 32m + 8*(2p+hf) .. +7 of token t
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int p = 0; p < 2; ++p) {
            const f32x16_p& a = acc[m][j];
            const uint32_t r0x = pack2<bf16>(a[8 * p + 0], a[8 * p + 1]);
            const uint32_t r0y = pack2<bf16>(a[8 * p + 2], a[8 * p + 3]);
            const uint32_t r1x = pack2<bf16>(a[8 * p + 4], a[8 * p + 5]);
            const uint32_t r1y = pack2<bf16>(a[8 * p + 6], a[8 * p + 7]);
            const auto sx = __builtin_amdgcn_permlane32_swap(r0x, r1x, false, false);
            const auto sy = __builtin_amdgcn_permlane32_swap(r0y, r1y, false, false);
            const int tc = 32 * m + 8 * (2 * p + hf);
            if (s0 + t < S)
              *reinterpret_cast<uint4*>(obase + (static_cast<int64_t>(tc / HD) * S + t) * HD + tc % HD) =
                  make_uint4(sx[0], sy[0], sx[1], sy[1]);
          }
      }
    };
    if (ntask < NW) {
      // One task per wave; the waves [ntask, NW) compute the QK-mean terms
      // and count themselves done in *qa_done, which a task wave waits for
      // (bounded: the counter only depends on waves that wait for nothing)
      // before its epilogue, so an early task (a short k head) does not wait
      // for the others.
      f32x16_p acc[MT][NT];
      if (wave < ntask) {
        mfma(wave, acc);
        if (qk_mean) {
          // Every lane of every term wave adds 1 with release order after
          // its own term writes; the acquire load that reads the final
          // count synchronises with all of those adds (one release
          // sequence), so the terms are visible to the epilogue's reads.
          const int want = 64 * (NW - ntask);
          bool ready = false;
          for (int spin = 0; spin < (1 << 22) && !ready; ++spin) {
            ready = __hip_atomic_load(qa_done, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= want;
            if (!ready) __builtin_amdgcn_s_sleep(2);
          }
          if (!ready) {
            // Cannot happen while the term waves run (they wait for
            // nothing); if it ever does, the tile's outputs become NaN and
            // the fault is counted for hydra_ccgqa_prep_faults, rather than
            // an epilogue over incomplete terms.
            if (lane == 0) atomicAdd(&g_prep_wait_faults, 1u);
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
              for (int j = 0; j < NT; ++j)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[m][j][i] = __builtin_nanf("");
          }
        }
        epilogue(wave, acc);
      } else {
        qa_work(ntask);
        __hip_atomic_fetch_add(qa_done, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        v_work(ntask);
      }
    } else {
      for (int task = wave; task < ntask; task += NW) {
        f32x16_p acc[MT][NT];
        mfma(task, acc);
        epilogue(task, acc);
      }
      const int extra = ntask % NW;  // waves with one task fewer write v
      if (wave >= extra) v_work(extra);
    }
  }
}

static size_t prep_mfma_lds(int64_t Hq, int64_t Hkv, int64_t hd, int TT) {
  const int64_t RS = (Hq + Hkv) * hd + 8;
  const int64_t nqa = Hq == Hkv ? Hq : 2;  // QK-mean terms per token
  return static_cast<size_t>(2 * TT + 6) * RS * 2 + static_cast<size_t>(TT) * (hd + 4) * 4 +
         static_cast<size_t>(TT) * (nqa * hd + 8) * 2 +
         static_cast<size_t>(((TT + 1) * (Hkv * hd + 8) + 7) / 8 * 8) * 2 + 16;
}

template <int HD>
static int launch_prep_mfma(const void* qkv, int64_t qkv_rs, const void* wq1, const void* wq2,
                            const void* wk1, const void* wk2, const void* temp, const float* cs,
                            const float* sn, int64_t cs_rs, void* qo, void* ko, void* vo,
                            int64_t B, int64_t S, int64_t Hq, int64_t Hkv, int flags,
                            size_t max_lds, hipStream_t st) {
  auto lds_for = [&](int TT) { return prep_mfma_lds(Hq, Hkv, HD, TT); };
  auto go = [&](auto tt_tag) -> int {
    constexpr int TT = decltype(tt_tag)::value;
    const size_t lds = lds_for(TT);
    auto kern = ccgqa_prep_mfma_kernel<HD, TT>;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) != hipSuccess)
      return fail(HYDRA_ERR_LAUNCH, "ccgqa_prep: cannot set the kernel's LDS size");
    const dim3 grid(static_cast<unsigned>((S + TT - 1) / TT), static_cast<unsigned>(B));
    kern<<<grid, kPrepThreads, lds, st>>>(
        static_cast<const bf16*>(qkv), qkv_rs, static_cast<const bf16*>(wq1),
        static_cast<const bf16*>(wq2), static_cast<const bf16*>(wk1),
        static_cast<const bf16*>(wk2), static_cast<const bf16*>(temp), cs, sn, cs_rs,
        static_cast<bf16*>(qo), static_cast<bf16*>(ko), static_cast<bf16*>(vo), (int)S,
        (int)Hq, (int)Hkv, flags);
    return check_launch("ccgqa_prep_mfma_kernel");
  };
  // 64-token tiles halve the weight traffic per MFMA; use them when they still
  // give at least one workgroup per CU (256), else 32-token tiles.
  int tt = B * ((S + 63) / 64) >= 256 ? 64 : 32;
  if (const char* e = getenv("HYDRA_PREP_TT")) tt = atoi(e) == 32 ? 32 : 64;
  if (tt == 64 && lds_for(64) <= max_lds) return go(std::integral_constant<int, 64>());
  if (lds_for(32) <= max_lds) return go(std::integral_constant<int, 32>());
  return -1;  // does not fit: caller falls back to the generic kernel
}

template <typename T>
static int launch_prep_vec(const void* qkv, int64_t qkv_rs, const void* wq1, const void* wq2,
                           const void* wk1, const void* wk2, const void* temp, const float* cs,
                           const float* sn, int64_t cs_rs, void* qo, void* ko, void* vo, int64_t B,
                           int64_t S, int64_t Hq, int64_t Hkv, int64_t hd, int flags,
                           size_t max_lds, hipStream_t st) {
  // 8-token tiles, or 4 when 8 would leave CUs without a workgroup (each
  // workgroup's time is mostly its weight reads, the same for both).
  const int64_t CW = (Hq + Hkv) * hd;
  const int tt = B * ((S + 7) / 8) < device_cus() ? 4 : 8;
  auto go = [&](auto tt_tag) -> int {
    constexpr int TT = decltype(tt_tag)::value;
    const size_t lds = static_cast<size_t>(3 * TT + 6) * CW * sizeof(float);
    if (lds > max_lds) return -1;
    auto kern = ccgqa_prep_vec_kernel<T, TT>;
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) != hipSuccess)
      return -1;
    const int threads = static_cast<int>(std::min<int64_t>(256, (CW + 63) / 64 * 64));
    const dim3 grid(static_cast<unsigned>((S + TT - 1) / TT), static_cast<unsigned>(B));
    kern<<<grid, threads, lds, st>>>(
        static_cast<const T*>(qkv), qkv_rs, static_cast<const T*>(wq1), static_cast<const T*>(wq2),
        static_cast<const T*>(wk1), static_cast<const T*>(wk2), static_cast<const T*>(temp), cs, sn,
        cs_rs, static_cast<T*>(qo), static_cast<T*>(ko), static_cast<T*>(vo), (int)S, (int)Hq,
        (int)Hkv, (int)hd, flags);
    return check_launch("ccgqa_prep_vec_kernel");
  };
  if (tt == 4) {
    const int rc = go(std::integral_constant<int, 4>());
    if (rc != -1) return rc;
  }
  return go(std::integral_constant<int, 8>());
}

template <typename T>
static int launch_prep_generic(const void* qkv, int64_t qkv_rs, const void* wq1,
                               const void* wq2, const void* wk1, const void* wk2,
                               const void* temp, const float* cs, const float* sn,
                               int64_t cs_rs, void* qo, void* ko, void* vo, int64_t B,
                               int64_t S, int64_t Hq, int64_t Hkv, int64_t hd, int64_t ks,
                               int flags, hipStream_t st) {
  const int64_t CW = (Hq + Hkv) * hd;
  const int64_t hw = ks - 1;  // token rows each causal conv reaches back
  auto lds_of = [&](int tt) { return static_cast<size_t>(3 * tt + 3 * hw) * CW * sizeof(T); };
  int TT = 32;
  while (TT > 1 && lds_of(TT) > 64 * 1024) TT >>= 1;
  const size_t lds = lds_of(TT);
  if (lds > 64 * 1024)
    return fail(HYDRA_ERR_UNSUPPORTED, "ccgqa_prep: latent too wide for the LDS tile");
  const dim3 grid(static_cast<unsigned>((S + TT - 1) / TT), static_cast<unsigned>(B));
  ccgqa_prep_generic_kernel<T><<<grid, 256, lds, st>>>(
      static_cast<const T*>(qkv), qkv_rs, static_cast<const T*>(wq1),
      static_cast<const T*>(wq2), static_cast<const T*>(wk1), static_cast<const T*>(wk2),
      static_cast<const T*>(temp), cs, sn, cs_rs, static_cast<T*>(qo), static_cast<T*>(ko),
      static_cast<T*>(vo), (int)S, (int)Hq, (int)Hkv, (int)hd, TT, (int)ks, flags);
  return check_launch("ccgqa_prep_generic_kernel");
}

}  // namespace hydra

using namespace hydra;

extern "C" int hydra_ccgqa_prep_faults(unsigned int* count) {
  if (!count) return hydra::fail(HYDRA_ERR_ARG, "hydra_ccgqa_prep_faults: null count");
  const hipError_t e = hipMemcpyFromSymbol(count, HIP_SYMBOL(hydra::g_prep_wait_faults), sizeof(unsigned int));
  if (e != hipSuccess) return hydra::fail(HYDRA_ERR_LAUNCH, std::string("hydra_ccgqa_prep_faults: ") + hipGetErrorString(e));
  return HYDRA_OK;
}

extern "C" int hydra_ccgqa_prep_tiled_ok(int64_t Hq, int64_t Hkv, int64_t hd, int dtype) {
  if (Hq < 1 || Hkv < 1 || Hq % Hkv != 0) return 0;
  if (dtype != HYDRA_BF16 || !(hd == 16 || hd == 32 || hd == 64 || hd == 128)) return 0;
  if ((Hq * hd) % 32 != 0 || (Hkv * hd) % 32 != 0) return 0;
  int dev = 0, max_lds = 65536;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
    max_lds = 65536;
  return prep_mfma_lds(Hq, Hkv, hd, 32) <= static_cast<size_t>(max_lds) ? 1 : 0;
}

extern "C" int hydra_ccgqa_prep_fwd(const void* qkv, int64_t qkv_rs, const void* wq1,
                                    const void* wq2, const void* wk1, const void* wk2,
                                    const void* temp, const float* cos, const float* sin,
                                    int64_t cs_rs, void* q_out, void* k_out, void* v_out,
                                    int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                                    int64_t hd, int64_t conv_ks, int flags, int dtype,
                                    void* stream) {
  HYDRA_REQUIRE(B >= 0 && S >= 0 && Hq >= 1 && Hkv >= 1 && hd >= 2, "ccgqa_prep: bad size");
  HYDRA_REQUIRE(conv_ks >= 1 && conv_ks <= 16, "ccgqa_prep: conv kernel size must be in [1, 16]");
  HYDRA_REQUIRE(Hq % Hkv == 0, "ccgqa_prep: n_heads must be a multiple of n_kv_heads");
  HYDRA_REQUIRE(hd % 2 == 0, "ccgqa_prep: head_dim must be even");
  HYDRA_REQUIRE((flags & ~127) == 0, "ccgqa_prep: unknown flag bits");
  const int64_t L = Hq * hd, K = Hkv * hd;
  HYDRA_REQUIRE(!(flags & HYDRA_CCGQA_VALUE_SHIFT) || K % 2 == 0,
                "ccgqa_prep: kv_dim must be even for the value shift");
  HYDRA_REQUIRE(qkv_rs >= L + 2 * K, "ccgqa_prep: qkv row stride smaller than L + 2K");
  if (B * S == 0) return HYDRA_OK;
  HYDRA_REQUIRE(qkv && q_out && k_out && v_out, "ccgqa_prep: null pointer");
  HYDRA_REQUIRE(!(flags & HYDRA_CCGQA_CONVS) || (wq1 && wq2 && wk1 && wk2),
                "ccgqa_prep: conv weights required");
  HYDRA_REQUIRE(!(flags & HYDRA_CCGQA_QK_NORM) || temp, "ccgqa_prep: temperature required");
  HYDRA_REQUIRE(!(flags & HYDRA_CCGQA_ROPE) || (cos && sin && cs_rs >= hd / 2),
                "ccgqa_prep: cos/sin [S, hd/2] required");
  HYDRA_REQUIRE(B <= 65535, "ccgqa_prep: batch must be <= 65535");
  HYDRA_REQUIRE(S * (L + 2 * K) < (int64_t(1) << 40), "ccgqa_prep: too large");
  auto st = static_cast<hipStream_t>(stream);
  const bool rope = flags & HYDRA_CCGQA_ROPE;
  // the MFMA and vector kernels are written for the reference's default
  // k = 3 (or no convs); other sizes take the generic kernel
  const bool k3 = conv_ks == 3 || !(flags & HYDRA_CCGQA_CONVS);
  const bool mfma_ok =
      k3 && dtype == HYDRA_BF16 && (hd == 16 || hd == 32 || hd == 64 || hd == 128) && K % 32 == 0 &&
      L % 32 == 0 &&
      qkv_rs % 8 == 0 && aligned16(qkv) && aligned16(q_out) && aligned16(k_out) &&
      aligned16(v_out) &&
      (!(flags & HYDRA_CCGQA_CONVS) || (aligned16(wq1) && aligned16(wq2) && aligned16(wk1) &&
                                        aligned16(wk2))) &&
      (!rope || (cs_rs % 4 == 0 && aligned16(cos) && aligned16(sin))) &&
      (!(flags & HYDRA_CCGQA_V_TRANSPOSED) || S % 8 == 0);
  if (mfma_ok) {
    int dev = 0, max_lds = 65536;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      max_lds = 65536;
    int rc = -1;
    switch (hd) {
      case 16: rc = launch_prep_mfma<16>(qkv, qkv_rs, wq1, wq2, wk1, wk2, temp, cos, sin, cs_rs, q_out, k_out, v_out, B, S, Hq, Hkv, flags, max_lds, st); break;
      case 32: rc = launch_prep_mfma<32>(qkv, qkv_rs, wq1, wq2, wk1, wk2, temp, cos, sin, cs_rs, q_out, k_out, v_out, B, S, Hq, Hkv, flags, max_lds, st); break;
      case 64: rc = launch_prep_mfma<64>(qkv, qkv_rs, wq1, wq2, wk1, wk2, temp, cos, sin, cs_rs, q_out, k_out, v_out, B, S, Hq, Hkv, flags, max_lds, st); break;
      default: rc = launch_prep_mfma<128>(qkv, qkv_rs, wq1, wq2, wk1, wk2, temp, cos, sin, cs_rs, q_out, k_out, v_out, B, S, Hq, Hkv, flags, max_lds, st); break;
    }
    if (rc >= 0) return rc;
  }
  if (flags & HYDRA_CCGQA_W_TILED)
    return fail(HYDRA_ERR_UNSUPPORTED,
                "ccgqa_prep: MFMA-tiled conv weights need the MFMA path (bf16, head_dim 16/32/64/128, "
                "16-byte aligned pointers, S % 8 == 0 with V_TRANSPOSED)");
  int dev = 0, max_lds = 65536;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
    max_lds = 65536;
  // 4-element weight and LDS steps: every channel count a multiple of 4.
  const int esz = dtype_size(dtype);
  const bool vec_ok = k3 && hd % 4 == 0 && aligned16(qkv) &&
                      (!(flags & HYDRA_CCGQA_CONVS) ||
                       ((reinterpret_cast<uintptr_t>(wq1) | reinterpret_cast<uintptr_t>(wq2) |
                         reinterpret_cast<uintptr_t>(wk1) | reinterpret_cast<uintptr_t>(wk2)) %
                            (4 * esz) == 0)) &&
                      getenv("HYDRA_PREP_GENERIC") == nullptr;
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    if (vec_ok) {
      const int rc = launch_prep_vec<T>(qkv, qkv_rs, wq1, wq2, wk1, wk2, temp, cos, sin, cs_rs,
                                        q_out, k_out, v_out, B, S, Hq, Hkv, hd, flags,
                                        static_cast<size_t>(max_lds), st);
      if (rc >= 0) return rc;
    }
    return launch_prep_generic<T>(qkv, qkv_rs, wq1, wq2, wk1, wk2, temp, cos, sin, cs_rs,
                                  q_out, k_out, v_out, B, S, Hq, Hkv, hd, conv_ks, flags, st);
  });
}
