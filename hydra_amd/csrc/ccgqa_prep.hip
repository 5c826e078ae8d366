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
// This is the generic (VALU, fp32 arithmetic) variant: any dtype, any even
// head_dim.  Conv weights are read in PyTorch Conv1d layout [out, in/groups, 3].
#include "common.h"

namespace hydra {

template <typename T>
__device__ __forceinline__ float rnd(float v) {
  return to_f32(from_f32<T>(v));
}

template <typename T>
__global__ __launch_bounds__(256) void ccgqa_prep_generic_kernel(
    const T* __restrict__ qkv, int64_t qkv_rs, const T* __restrict__ wq1,
    const T* __restrict__ wq2, const T* __restrict__ wk1, const T* __restrict__ wk2,
    const T* __restrict__ temp, const float* __restrict__ cs, const float* __restrict__ sn,
    int64_t cs_rs, T* __restrict__ qo, T* __restrict__ ko, T* __restrict__ vo, int S,
    int Hq, int Hkv, int hd, int TT, int flags) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  T* sm = reinterpret_cast<T*>(smem_raw);
  const int L = Hq * hd, K = Hkv * hd, CW = L + K;
  T* xs = sm;                        // rows: tokens s0-4 .. s0+TT-1
  T* y1 = xs + (TT + 4) * CW;        // rows: tokens s0-2 .. s0+TT-1
  T* y2 = y1 + (TT + 2) * CW;        // rows: tokens s0   .. s0+TT-1
  const int tid = threadIdx.x;
  const int b = blockIdx.y;
  const int s0 = blockIdx.x * TT;
  const bool convs = flags & HYDRA_CCGQA_CONVS;
  const bool qk_mean = flags & HYDRA_CCGQA_QK_MEAN;
  const bool vshift = flags & HYDRA_CCGQA_VALUE_SHIFT;
  const bool qk_norm = flags & HYDRA_CCGQA_QK_NORM;
  const bool rope = flags & HYDRA_CCGQA_ROPE;
  const T* xb = qkv + static_cast<int64_t>(b) * S * qkv_rs;

  for (int i = tid; i < (TT + 4) * CW; i += 256) {
    const int r = i / CW, c = i - r * CW;
    const int s = s0 - 4 + r;
    xs[i] = (s >= 0 && s < S) ? xb[static_cast<int64_t>(s) * qkv_rs + c] : from_f32<T>(0.f);
  }
  __syncthreads();

  if (convs) {
    // conv1 (grouped): output channel o of group g reads channels g*hd..g*hd+hd-1.
    for (int i = tid; i < (TT + 2) * CW; i += 256) {
      const int r = i / CW, o = i - r * CW;
      const int s = s0 - 2 + r;
      float acc = 0.f;
      if (s >= 0 && s < S) {
        const bool is_q = o < L;
        const int oo = is_q ? o : o - L;
        const int col0 = (is_q ? 0 : L) + (oo / hd) * hd;
        const T* w = (is_q ? wq1 : wk1) + static_cast<int64_t>(oo) * hd * 3;
        for (int t = 0; t < 3; ++t) {
          const T* xr = xs + (r + t) * CW + col0;
          for (int c = 0; c < hd; ++c) acc = fmaf(to_f32(w[c * 3 + t]), to_f32(xr[c]), acc);
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
      const T* w = (is_q ? wq2 : wk2) + static_cast<int64_t>(oo) * C * 3;
      float acc = 0.f;
      for (int t = 0; t < 3; ++t) {
        const T* yr = y1 + (r + t) * CW + col0;
        for (int c = 0; c < C; ++c) acc = fmaf(to_f32(w[c * 3 + t]), to_f32(yr[c]), acc);
      }
      y2[i] = from_f32<T>(acc);
    }
  } else {
    for (int i = tid; i < TT * CW; i += 256) y2[i] = xs[4 * CW + i];
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
    const T* x0 = xs + (r + 4) * CW;  // pre-conv q0 | k0 of this token
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
    vo[((static_cast<int64_t>(b) * Hkv + j) * S + s) * hd + d] = val;
  }
}

template <typename T>
static int launch_prep_generic(const void* qkv, int64_t qkv_rs, const void* wq1,
                               const void* wq2, const void* wk1, const void* wk2,
                               const void* temp, const float* cs, const float* sn,
                               int64_t cs_rs, void* qo, void* ko, void* vo, int64_t B,
                               int64_t S, int64_t Hq, int64_t Hkv, int64_t hd, int flags,
                               hipStream_t st) {
  const int64_t CW = (Hq + Hkv) * hd;
  int TT = 32;
  while (TT > 1 && static_cast<int64_t>(3 * TT + 6) * CW * sizeof(T) > 64 * 1024) TT >>= 1;
  const size_t lds = static_cast<size_t>(3 * TT + 6) * CW * sizeof(T);
  if (lds > 64 * 1024)
    return fail(HYDRA_ERR_UNSUPPORTED, "ccgqa_prep: latent too wide for the LDS tile");
  const dim3 grid(static_cast<unsigned>((S + TT - 1) / TT), static_cast<unsigned>(B));
  ccgqa_prep_generic_kernel<T><<<grid, 256, lds, st>>>(
      static_cast<const T*>(qkv), qkv_rs, static_cast<const T*>(wq1),
      static_cast<const T*>(wq2), static_cast<const T*>(wk1), static_cast<const T*>(wk2),
      static_cast<const T*>(temp), cs, sn, cs_rs, static_cast<T*>(qo), static_cast<T*>(ko),
      static_cast<T*>(vo), (int)S, (int)Hq, (int)Hkv, (int)hd, TT, flags);
  return check_launch("ccgqa_prep_generic_kernel");
}

}  // namespace hydra

using namespace hydra;

extern "C" int hydra_ccgqa_prep_fwd(const void* qkv, int64_t qkv_rs, const void* wq1,
                                    const void* wq2, const void* wk1, const void* wk2,
                                    const void* temp, const float* cos, const float* sin,
                                    int64_t cs_rs, void* q_out, void* k_out, void* v_out,
                                    int64_t B, int64_t S, int64_t Hq, int64_t Hkv,
                                    int64_t hd, int flags, int dtype, void* stream) {
  HYDRA_REQUIRE(B >= 0 && S >= 0 && Hq >= 1 && Hkv >= 1 && hd >= 2, "ccgqa_prep: bad size");
  HYDRA_REQUIRE(Hq % Hkv == 0, "ccgqa_prep: n_heads must be a multiple of n_kv_heads");
  HYDRA_REQUIRE(hd % 2 == 0, "ccgqa_prep: head_dim must be even");
  HYDRA_REQUIRE((flags & ~31) == 0, "ccgqa_prep: unknown flag bits");
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
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    return launch_prep_generic<T>(qkv, qkv_rs, wq1, wq2, wk1, wk2, temp, cos, sin, cs_rs,
                                  q_out, k_out, v_out, B, S, Hq, Hkv, hd, flags, st);
  });
}
