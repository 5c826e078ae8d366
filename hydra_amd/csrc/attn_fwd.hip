// CCGQA attention core on gfx950: causal (or full) GQA softmax attention
// forward, o = softmax(scale * q k^T + mask) v, with K/V heads shared by
// G = Hq/Hkv query heads in repeat_interleave order.
// Reference semantics: SDPA call of CCGQAAttention.forward
// (hydra/attention/backends/ccgqa/attention.py:268-327) and the Triton
// kernels _fwd_gqa_kernel / _fwd_kernel (kernels/fused_attention.py:14-110,
// 341-429).
//
// bf16 path (attn_fwd_mfma_kernel): v_mfma_f32_32x32x16_bf16.
//  * A workgroup is NW waves (4, or 2 when that is needed to give the
//    dispatcher enough workgroups to balance the causal triangle) that share
//    one (batch, kv-head) and one staged K/V tile in LDS; wave w takes task
//    NW*wg+w, task t -> (32-row query block t/G, query head kvh*G + t%G), so
//    GQA heads reuse the same K/V tile.
//  * Scores are computed transposed, S^T = K Q^T, so lane l owns query
//    (l%32) and the online softmax needs no cross-lane traffic except one
//    swap between the two half-waves.
//  * O^T = V^T P^T: the bf16 P fragment is taken straight from the score
//    accumulator registers; V is transposed while it is staged into LDS.
//  * Softmax runs in the exp2 domain with fp32 statistics; the scale is
//    folded into one FMA per score, and the running max (with the O
//    rescale it implies) only moves when a tile's max exceeds it by 2^8.
//  * K/V tiles are double-buffered in LDS: one barrier per key tile, the
//    global loads of tile j+1 are in flight while tile j is computed.
//  * Causal: the grid runs the longest query blocks first (with the second
//    half of the grid in reverse, so co-resident workgroups balance), blocks
//    above the diagonal are skipped, only diagonal tiles evaluate the mask.
// Generic path (attn_fwd_generic_kernel): one thread per query row, fp32
// math, any element type, even head_dim <= 256.
#include "common.h"

#include <cstdlib>
#include <type_traits>

namespace hydra {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
constexpr uint32_t kOnesBf16x2 = 0x3f803f80u;  // (1.0, 1.0) in bf16

// acc + a.lo*b.lo + a.hi*b.hi on packed bf16 pairs (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}


template <int HD, bool CAUSAL, int MASK, bool VT, int NW>
__global__ __launch_bounds__(64 * NW) void attn_fwd_mfma_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    bf16* __restrict__ o, float* __restrict__ lse, const uint8_t* __restrict__ kmask,
    int S, int Hq, int Hkv, int G, int ntasks, int nwg,
    int64_t qs0, int64_t qs1, int64_t qs2,
    int64_t ks0, int64_t ks1, int64_t ks2,
    int64_t vs0, int64_t vs1, int64_t vs2,
    int64_t os0, int64_t os1, int64_t os2, float scale_log2) {
  // VT: V is stored transposed ([.., hd, S], keys contiguous, row stride
  // vs2 between d rows) and is staged with plain 16-byte copies; otherwise
  // V is [.., S, hd] and is transposed while staged.
  constexpr int BN = 64;                // keys per tile
  constexpr int KSTEPS = HD / 16;       // k-steps of S^T = K Q^T
  constexpr int DT = (HD + 31) / 32;    // 32-row d tiles of O^T
  constexpr int KROW = HD + 8;          // padded LDS row of K (elements)
  constexpr int VROW = BN + 4;          // padded LDS row of V^T (elements)
  constexpr int DC = HD / 8;            // 16-byte chunks per K/V row
  constexpr int NT = 64 * NW;                       // threads per workgroup
  constexpr int KCH = (BN * DC + NT - 1) / NT;      // K chunks per thread
  constexpr int VCH = ((BN / 2) * DC + NT - 1) / NT;  // V key-pair units per thread
  constexpr int KBUF = BN * KROW, VBUF = DT * 32 * VROW;
  // Lazy rescaling: the running max used for exp2 only moves when a score
  // exceeds it by more than this (log2 units), so P stays <= 2^8.
  constexpr float kRescale = 8.f;

  __shared__ __attribute__((aligned(16))) uint16_t Ks[2 * KBUF];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2 * VBUF];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n = lane & 31, hf = lane >> 5;
  // Causal balance: workgroups are ranked by work (longest first) and the
  // second half of the grid takes the ranks in reverse, so the two
  // workgroups that share a CU carry complementary amounts of work.
  const int BH = gridDim.x / nwg;
  const int total = gridDim.x;
  const int half = (total + 1) / 2;
  const int pos = blockIdx.x;
  const int rank = pos < half ? pos : total - 1 - (pos - half);
  const int wg = nwg - 1 - rank / BH;
  const int bk = rank - (rank / BH) * BH;
  const int b = bk / Hkv, kvh = bk - b * Hkv;
  const int task = wg * NW + wave;
  const bool active = task < ntasks;
  const int qb = task / G;
  const int h = kvh * G + (task - qb * G);
  const int q0 = qb * 32;
  const int qi = q0 + n;
  const int last_task = min(wg * NW + NW - 1, ntasks - 1);
  const int wg_qmax = (last_task / G) * 32 + 31;
  const int kend = (CAUSAL && MASK != 2) ? min(S, wg_qmax + 1) : S;
  const int nkb = (kend + BN - 1) / BN;

  const bf16* kbase = k + b * ks0 + kvh * ks1;
  const bf16* vbase = v + b * vs0 + kvh * vs1;

  if (DT * 32 > HD) {  // zero the padding rows of both V^T buffers once
    for (int i = tid; i < (DT * 32 - HD) * VROW; i += NT) {
      Vt[HD * VROW + i] = 0;
      Vt[VBUF + HD * VROW + i] = 0;
    }
  }

  // Q fragments (B operand of S^T = K Q^T): lane holds q[qi, 16s+8hf .. +7].
  bf16x8_t qf[KSTEPS];
  {
    const bf16* qrow = q + b * qs0 + h * qs1 + static_cast<int64_t>(qi) * qs2;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (active && qi < S) raw = *reinterpret_cast<const uint4*>(qrow + 16 * s + 8 * hf);
      qf[s] = as_bf16x8(raw);
    }
  }

  // Retire the Q loads here: otherwise the in-order vmcnt makes the first
  // MFMA of every iteration wait for the next tile's prefetch as well.
  __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)

  constexpr int VTCH = (HD * (BN / 8) + NT - 1) / NT;  // V^T 16-byte chunks per thread
  uint4 kreg[KCH];
  uint4 vreg[VT ? VTCH : VCH][2];
  // Global -> registers for the tile at key0.  FULL tiles (key0 + BN <= S)
  // skip the per-row bounds tests.
  auto fetch = [&](int key0, auto full_tag) {
    constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int c = tid + NT * j;
      const int key = c / DC, dc = c - key * DC;
      if (FULL && (BN * DC) % NT == 0) {
        kreg[j] = *reinterpret_cast<const uint4*>(kbase + static_cast<int64_t>(key0 + key) * ks2 + dc * 8);
      } else {
        kreg[j] = make_uint4(0, 0, 0, 0);
        if (c < BN * DC && (FULL || key0 + key < S))
          kreg[j] = *reinterpret_cast<const uint4*>(kbase + static_cast<int64_t>(key0 + key) * ks2 + dc * 8);
      }
    }
    if constexpr (VT) {
#pragma unroll
      for (int j = 0; j < VTCH; ++j) {
        const int c = tid + NT * j;
        const int d = c / (BN / 8), kc = c - d * (BN / 8);
        vreg[j][0] = make_uint4(0, 0, 0, 0);
        // S % 8 == 0 on this path, so a chunk is either fully in or out
        if (c < HD * (BN / 8) && (FULL || key0 + 8 * kc < S))
          vreg[j][0] = *reinterpret_cast<const uint4*>(vbase + static_cast<int64_t>(d) * vs2 + key0 + 8 * kc);
      }
    } else {
#pragma unroll
      for (int j = 0; j < VCH; ++j) {
        const int u = tid + NT * j;
        const int kp = u / DC, dc = u - kp * DC;
        const int key = key0 + 2 * kp;
        vreg[j][0] = make_uint4(0, 0, 0, 0);
        vreg[j][1] = make_uint4(0, 0, 0, 0);
        if (u < (BN / 2) * DC) {
          if (FULL || key < S) vreg[j][0] = *reinterpret_cast<const uint4*>(vbase + static_cast<int64_t>(key) * vs2 + dc * 8);
          if (FULL || key + 1 < S) vreg[j][1] = *reinterpret_cast<const uint4*>(vbase + static_cast<int64_t>(key + 1) * vs2 + dc * 8);
        }
      }
    }
  };
  auto fetch_tile = [&](int key0) {
    if (key0 + BN <= S) fetch(key0, std::true_type());
    else fetch(key0, std::false_type());
  };
  auto stage = [&](int buf) {
    uint16_t* kd = Ks + buf * KBUF;
    uint16_t* vd = Vt + buf * VBUF;
#pragma unroll
    for (int j = 0; j < KCH; ++j) {
      const int c = tid + NT * j;
      const int key = c / DC, dc = c - key * DC;
      if (c < BN * DC) *reinterpret_cast<uint4*>(&kd[key * KROW + dc * 8]) = kreg[j];
    }
    if constexpr (VT) {
#pragma unroll
      for (int j = 0; j < VTCH; ++j) {
        const int c = tid + NT * j;
        const int d = c / (BN / 8), kc = c - d * (BN / 8);
        if (c < HD * (BN / 8)) {
          // VROW*2 bytes is a multiple of 8, not of 16: two 8-byte stores
          *reinterpret_cast<uint2*>(&vd[d * VROW + 8 * kc]) = make_uint2(vreg[j][0].x, vreg[j][0].y);
          *reinterpret_cast<uint2*>(&vd[d * VROW + 8 * kc + 4]) = make_uint2(vreg[j][0].z, vreg[j][0].w);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < VCH; ++j) {
        const int u = tid + NT * j;
        const int kp = u / DC, dc = u - kp * DC;
        if (u < (BN / 2) * DC) {
          const uint32_t a[4] = {vreg[j][0].x, vreg[j][0].y, vreg[j][0].z, vreg[j][0].w};
          const uint32_t c2[4] = {vreg[j][1].x, vreg[j][1].y, vreg[j][1].z, vreg[j][1].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // d = dc*8 + 2e (low halves) and d+1 (high halves); keys 2kp, 2kp+1
            const uint32_t lo = __builtin_amdgcn_perm(c2[e], a[e], 0x05040100u);
            const uint32_t hi = __builtin_amdgcn_perm(c2[e], a[e], 0x07060302u);
            *reinterpret_cast<uint32_t*>(&vd[(dc * 8 + 2 * e) * VROW + 2 * kp]) = lo;
            *reinterpret_cast<uint32_t*>(&vd[(dc * 8 + 2 * e + 1) * VROW + 2 * kp]) = hi;
          }
        }
      }
    }
  };

  float m_i = -INFINITY, l_i = 0.f;
  f32x16_t acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;

  // One key tile: S^T = K Q^T, online softmax, O^T += V^T P^T.  MASKED is
  // compile-time, so the tiles that are fully visible to every wave of the
  // workgroup run with no mask code at all.
  auto tile = [&](int kb, auto masked_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    const int buf = kb & 1;
    const int key0 = kb * BN;
    const uint16_t* kt = Ks + buf * KBUF;
    const uint16_t* vt = Vt + buf * VBUF;
    f32x16_t st[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) st[mt][r] = 0.f;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const uint4 a = *reinterpret_cast<const uint4*>(&kt[(32 * mt + n) * KROW + 16 * s + 8 * hf]);
        st[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), qf[s], st[mt], 0, 0, 0);
      }
    if constexpr (MASKED) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = key0 + 32 * mt + 8 * (r >> 2) + 4 * hf + (r & 3);
          bool ok = key < S;
          if (CAUSAL && MASK != 2) ok = ok && key <= qi;
          if (MASK != 0) {
            const bool keep = kmask[static_cast<int64_t>(b) * S + min(key, S - 1)] != 0;
            ok = ok && (MASK == 1 ? keep : (key > qi || !keep));
          }
          st[mt][r] = ok ? st[mt][r] : -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[mt][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32)) * scale_log2;  // scaled row max of this tile
    // Move the reference max only when this tile would push P past 2^8; the
    // test is made wave-uniform so the common case is one skipped branch.
    if (__any(mx > m_i + kRescale)) {
      const bool move = mx > m_i + kRescale;
      // alpha = 0 when m_i = -inf; lanes that keep their max (including rows
      // with no visible key yet, where m_i - m_i would be NaN) keep alpha = 1.
      const float alpha = move ? __builtin_amdgcn_exp2f(m_i - mx) : 1.f;
      const float m_new = move ? mx : m_i;
      l_i *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[dt][r] *= alpha;
      m_i = m_new;
    }
    const float m_use = m_i == -INFINITY ? 0.f : m_i;
    // P in bf16, and its row sum from the same rounded values (v_dot2 with
    // (1, 1)), so the normalisation uses exactly the P of the PV product.
    uint4 pk[4];
    float rs = 0.f;
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
      const int mt = s2 >> 1, rb = 8 * (s2 & 1);
      float p[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        p[e] = __builtin_amdgcn_exp2f(fmaf(st[mt][rb + e], scale_log2, -m_use));
      pk[s2].x = pack2<bf16>(p[0], p[1]);
      pk[s2].y = pack2<bf16>(p[2], p[3]);
      pk[s2].z = pack2<bf16>(p[4], p[5]);
      pk[s2].w = pack2<bf16>(p[6], p[7]);
      rs = dot2_bf16(pk[s2].x, kOnesBf16x2, rs);
      rs = dot2_bf16(pk[s2].y, kOnesBf16x2, rs);
      rs = dot2_bf16(pk[s2].z, kOnesBf16x2, rs);
      rs = dot2_bf16(pk[s2].w, kOnesBf16x2, rs);
    }
    l_i += rs + __shfl_xor(rs, 32);
    // O^T += V^T P^T over 4 k-steps of 16 keys.
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2) {
      const bf16x8_t pf = as_bf16x8(pk[s2]);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint16_t* vr = &vt[(32 * dt + n) * VROW + 16 * s2 + 4 * hf];
        const uint2 lo = *reinterpret_cast<const uint2*>(vr);
        const uint2 hi = *reinterpret_cast<const uint2*>(vr + 8);
        const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), pf, acc[dt], 0, 0, 0);
      }
    }
  };

  // Tiles [0, nfull) are in bounds and at or below the diagonal of every
  // wave of the workgroup; the rest need the mask.
  const int wg_qmin = ((wg * NW) / G) * 32;
  int nfull = 0;
  if (MASK == 0) nfull = min(CAUSAL ? (wg_qmin + 1) / BN : nkb, S / BN);
  nfull = min(nfull, nkb);

  if (nkb > 0) {
    fetch_tile(0);
    stage(0);
  }
  __syncthreads();
  int kb = 0;
  for (; kb < nfull; ++kb) {
    if (kb + 1 < nkb) fetch_tile((kb + 1) * BN);
    if (active) tile(kb, std::false_type());
    // The next tile goes into the other buffer, which every wave finished
    // reading before the barrier that ended the previous iteration.
    if (kb + 1 < nkb) stage((kb & 1) ^ 1);
    __syncthreads();
  }
  for (; kb < nkb; ++kb) {
    if (kb + 1 < nkb) fetch_tile((kb + 1) * BN);
    const bool live = active && !(CAUSAL && MASK != 2 && kb * BN > q0 + 31);
    if (live) tile(kb, std::true_type());
    if (kb + 1 < nkb) stage((kb & 1) ^ 1);
    __syncthreads();
  }

  if (!active || qi >= S) return;
  const float inv = l_i > 0.f ? 1.f / l_i : 0.f;
  bf16* orow = o + b * os0 + h * os1 + static_cast<int64_t>(qi) * os2;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d = 32 * dt + 8 * g4 + 4 * hf;
      if (d < HD) {
        uint2 w;
        w.x = pack2<bf16>(acc[dt][4 * g4 + 0] * inv, acc[dt][4 * g4 + 1] * inv);
        w.y = pack2<bf16>(acc[dt][4 * g4 + 2] * inv, acc[dt][4 * g4 + 3] * inv);
        *reinterpret_cast<uint2*>(orow + d) = w;
      }
    }
  if (lse && hf == 0) {
    lse[(static_cast<int64_t>(b) * Hq + h) * S + qi] =
        l_i > 0.f ? (m_i + __log2f(l_i)) * kLn2 : -INFINITY;
  }
}

// ---- generic path ---------------------------------------------------------
template <typename T, int MAXHD>
__global__ __launch_bounds__(256) void attn_fwd_generic_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    T* __restrict__ o, float* __restrict__ lse, const uint8_t* __restrict__ kmask,
    int B, int S, int Hq, int Hkv, int hd, int causal, int mask_mode,
    int64_t qs0, int64_t qs1, int64_t qs2, int64_t ks0, int64_t ks1, int64_t ks2,
    int64_t vs0, int64_t vs1, int64_t vs2, int64_t vs3, int64_t os0, int64_t os1, int64_t os2,
    float scale) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= static_cast<int64_t>(B) * Hq * S) return;
  const int s = static_cast<int>(gid % S);
  const int bh = static_cast<int>(gid / S);
  const int b = bh / Hq, h = bh - b * Hq;
  const int j = h / (Hq / Hkv);
  float qv[MAXHD], acc[MAXHD];
  const T* qr = q + b * qs0 + h * qs1 + static_cast<int64_t>(s) * qs2;
  for (int d = 0; d < hd; ++d) {
    qv[d] = to_f32(qr[d]);
    acc[d] = 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int tend = (causal && mask_mode != 2) ? s + 1 : S;
  const T* kb = k + b * ks0 + j * ks1;
  const T* vb = v + b * vs0 + j * vs1;
  for (int t = 0; t < tend; ++t) {
    if (mask_mode == 1 && kmask[static_cast<int64_t>(b) * S + t] == 0) continue;
    if (mask_mode == 2 && t <= s && kmask[static_cast<int64_t>(b) * S + t] != 0) continue;
    const T* kr = kb + static_cast<int64_t>(t) * ks2;
    float dot = 0.f;
    for (int d = 0; d < hd; ++d) dot = fmaf(qv[d], to_f32(kr[d]), dot);
    const float x = dot * scale;
    if (x > m) {
      const float alpha = expf(m - x);
      for (int d = 0; d < hd; ++d) acc[d] *= alpha;
      l *= alpha;
      m = x;
    }
    const float p = expf(x - m);
    l += p;
    const T* vr = vb + static_cast<int64_t>(t) * vs2;
    for (int d = 0; d < hd; ++d) acc[d] = fmaf(p, to_f32(vr[d * vs3]), acc[d]);
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  T* orow = o + b * os0 + h * os1 + static_cast<int64_t>(s) * os2;
  for (int d = 0; d < hd; ++d) orow[d] = from_f32<T>(acc[d] * inv);
  if (lse) lse[gid] = l > 0.f ? m + logf(l) : -INFINITY;
}

template <int HD>
static int launch_mfma(const void* q, const void* k, const void* v, void* o, float* lse,
                       const uint8_t* kmask, int mask_mode, int64_t B, int64_t Hq,
                       int64_t Hkv, int64_t S, const int64_t* qs, const int64_t* ks,
                       const int64_t* vs, const int64_t* os, bool causal, float scale,
                       hipStream_t st) {
  // V with unit stride along the keys is read as V^T rows (vs[3] apart).
  const bool vt = vs[2] == 1 && vs[3] != 1;
  const int G = static_cast<int>(Hq / Hkv);
  const int nqb = static_cast<int>((S + 31) / 32);
  const int ntasks = G * nqb;
  // Four-wave workgroups share each staged K/V tile between four query
  // blocks; two-wave ones (HYDRA_ATTN_NW=2) halve that reuse and measured
  // slower even where they double the workgroup count.
  int nw = 4;
  if (const char* e = getenv("HYDRA_ATTN_NW")) nw = atoi(e) == 2 ? 2 : 4;
  const int nwg = (ntasks + nw - 1) / nw;
  const dim3 grid(static_cast<unsigned>(nwg * B * Hkv));
  const float sl2 = scale * kLog2e;
  auto Q = static_cast<const bf16*>(q);
  auto K = static_cast<const bf16*>(k);
  auto V = static_cast<const bf16*>(v);
  auto O = static_cast<bf16*>(o);
  auto go = [&](auto c_tag, auto m_tag, auto nw_tag) {
    constexpr bool C = decltype(c_tag)::value;
    constexpr int M = decltype(m_tag)::value;
    constexpr int NW = decltype(nw_tag)::value;
    if (vt)
      attn_fwd_mfma_kernel<HD, C, M, true, NW><<<grid, 64 * NW, 0, st>>>(
          Q, K, V, O, lse, kmask, (int)S, (int)Hq, (int)Hkv, G, ntasks, nwg, qs[0], qs[1],
          qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[3], os[0], os[1], os[2], sl2);
    else
      attn_fwd_mfma_kernel<HD, C, M, false, NW><<<grid, 64 * NW, 0, st>>>(
          Q, K, V, O, lse, kmask, (int)S, (int)Hq, (int)Hkv, G, ntasks, nwg, qs[0], qs[1],
          qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], os[0], os[1], os[2], sl2);
  };
  auto by_nw = [&](auto c_tag, auto m_tag) {
    if (nw == 2) go(c_tag, m_tag, std::integral_constant<int, 2>());
    else go(c_tag, m_tag, std::integral_constant<int, 4>());
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  using M0 = std::integral_constant<int, 0>;
  using M1 = std::integral_constant<int, 1>;
  using M2 = std::integral_constant<int, 2>;
  // The reference-SDPA mask mode opens keys above the diagonal, so it walks
  // every key tile (no causal tile skipping).
  if (mask_mode == HYDRA_MASK_REFERENCE_SDPA) by_nw(F_(), M2());
  else if (causal && mask_mode == HYDRA_MASK_KEY_PADDING) by_nw(T_(), M1());
  else if (causal) by_nw(T_(), M0());
  else if (mask_mode == HYDRA_MASK_KEY_PADDING) by_nw(F_(), M1());
  else by_nw(F_(), M0());
  return check_launch("attn_fwd_mfma_kernel");
}

template <typename T>
static int launch_generic(const void* q, const void* k, const void* v, void* o, float* lse,
                          const uint8_t* kmask, int mask_mode, int64_t B, int64_t Hq,
                          int64_t Hkv, int64_t S, int64_t hd, const int64_t* qs,
                          const int64_t* ks, const int64_t* vs, const int64_t* os,
                          bool causal, float scale, hipStream_t st) {
  const int64_t total = B * Hq * S;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  auto Q = static_cast<const T*>(q);
  auto K = static_cast<const T*>(k);
  auto V = static_cast<const T*>(v);
  auto O = static_cast<T*>(o);
#define HYDRA_GEN_LAUNCH(MAXHD)                                                       \
  attn_fwd_generic_kernel<T, MAXHD><<<grid, 256, 0, st>>>(                            \
      Q, K, V, O, lse, kmask, (int)B, (int)S, (int)Hq, (int)Hkv, (int)hd, causal ? 1 : 0, \
      mask_mode, qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], vs[3], os[0], \
      os[1], os[2], scale)
  if (hd <= 32) HYDRA_GEN_LAUNCH(32);
  else if (hd <= 64) HYDRA_GEN_LAUNCH(64);
  else if (hd <= 128) HYDRA_GEN_LAUNCH(128);
  else HYDRA_GEN_LAUNCH(256);
#undef HYDRA_GEN_LAUNCH
  return check_launch("attn_fwd_generic_kernel");
}

}  // namespace hydra

using namespace hydra;

extern "C" int hydra_attn_fwd(const void* q, const void* k, const void* v, void* o,
                              float* lse, const uint8_t* key_mask, int mask_mode,
                              int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t hd,
                              const int64_t* qs, const int64_t* ks, const int64_t* vs,
                              const int64_t* os, int causal, float scale, int dtype,
                              void* stream) {
  HYDRA_REQUIRE(B >= 0 && S >= 0 && Hq >= 1 && Hkv >= 1 && hd >= 1, "attn_fwd: bad size");
  HYDRA_REQUIRE(Hq % Hkv == 0, "attn_fwd: n_heads must be a multiple of n_kv_heads");
  HYDRA_REQUIRE(qs && ks && vs && os, "attn_fwd: null stride array");
  HYDRA_REQUIRE(qs[3] == 1 && ks[3] == 1 && os[3] == 1,
                "attn_fwd: q, k and o must have unit stride along head_dim");
  HYDRA_REQUIRE(vs[3] == 1 || vs[2] == 1,
                "attn_fwd: v needs unit stride along head_dim or along the sequence");
  HYDRA_REQUIRE(hd <= 256, "attn_fwd: head_dim must be <= 256");
  HYDRA_REQUIRE(mask_mode >= HYDRA_MASK_NONE && mask_mode <= HYDRA_MASK_REFERENCE_SDPA,
                "attn_fwd: unknown mask mode");
  HYDRA_REQUIRE(mask_mode == HYDRA_MASK_NONE || key_mask != nullptr,
                "attn_fwd: mask mode needs key_mask");
  HYDRA_REQUIRE(mask_mode != HYDRA_MASK_REFERENCE_SDPA || causal,
                "attn_fwd: the reference-SDPA mask mode is defined with causal=1");
  if (B * S == 0) return HYDRA_OK;
  HYDRA_REQUIRE(q && k && v && o, "attn_fwd: null pointer");
  HYDRA_REQUIRE(S < (int64_t(1) << 30), "attn_fwd: sequence too long");
  HYDRA_REQUIRE(B * Hkv * ((Hq / Hkv) * ((S + 31) / 32) + 3) / 4 < (int64_t(1) << 31),
                "attn_fwd: too many workgroups");
  const uint8_t* km = mask_mode == HYDRA_MASK_NONE ? nullptr : key_mask;
  auto st = static_cast<hipStream_t>(stream);
  const bool mfma_shape = (hd == 16 || hd == 32 || hd == 64 || hd == 128);
  bool strides8 = true;
  for (int i = 0; i < 3; ++i)
    strides8 = strides8 && qs[i] % 8 == 0 && ks[i] % 8 == 0 && os[i] % 4 == 0;
  if (vs[3] == 1) {
    strides8 = strides8 && vs[0] % 8 == 0 && vs[1] % 8 == 0 && vs[2] % 8 == 0;
  } else {  // V^T rows: 16-byte chunks of 8 keys, so S must be a multiple of 8
    strides8 = strides8 && vs[0] % 8 == 0 && vs[1] % 8 == 0 && vs[3] % 8 == 0 && S % 8 == 0;
  }
  if (dtype == HYDRA_BF16 && mfma_shape && strides8 && aligned16(q) && aligned16(k) &&
      aligned16(v) && (reinterpret_cast<uintptr_t>(o) & 7u) == 0) {
    switch (hd) {
      case 16: return launch_mfma<16>(q, k, v, o, lse, km, mask_mode, B, Hq, Hkv, S, qs, ks, vs, os, causal != 0, scale, st);
      case 32: return launch_mfma<32>(q, k, v, o, lse, km, mask_mode, B, Hq, Hkv, S, qs, ks, vs, os, causal != 0, scale, st);
      case 64: return launch_mfma<64>(q, k, v, o, lse, km, mask_mode, B, Hq, Hkv, S, qs, ks, vs, os, causal != 0, scale, st);
      default: return launch_mfma<128>(q, k, v, o, lse, km, mask_mode, B, Hq, Hkv, S, qs, ks, vs, os, causal != 0, scale, st);
    }
  }
  HYDRA_REQUIRE(B * Hq * S / 256 < (int64_t(1) << 31), "attn_fwd: too many rows");
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    return launch_generic<T>(q, k, v, o, lse, km, mask_mode, B, Hq, Hkv, S, hd, qs, ks, vs,
                             os, causal != 0, scale, st);
  });
}
