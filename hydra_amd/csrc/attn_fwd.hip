// CCGQA attention core on gfx950: causal (or full) GQA softmax attention
// forward, o = softmax(scale * q k^T + mask) v, with K/V heads shared by
// G = Hq/Hkv query heads in repeat_interleave order.
// Reference semantics: SDPA call of CCGQAAttention.forward
// (hydra/attention/backends/ccgqa/attention.py:268-327) and the Triton
// kernels _fwd_gqa_kernel / _fwd_kernel (kernels/fused_attention.py:14-110,
// 341-429).
//
// bf16 path (attn_fwd_mfma_kernel): v_mfma_f32_32x32x16_bf16.
//  * A workgroup is 4 waves that share one (batch, kv-head) and one staged
//    K/V tile in LDS; an item is 4 query tasks, task t -> (32-row query
//    block t/G, query head kvh*G + t%G), so GQA heads reuse the same tile.
//  * Scores are computed transposed, S^T = K Q^T, so lane l owns query
//    (l%32) and the online softmax needs no cross-lane traffic except one
//    swap between the two half-waves (v_permlane32_swap).
//  * O^T = V^T P^T: the bf16 P fragment is taken straight from the score
//    accumulator registers; V is transposed while it is staged into LDS,
//    or read as V^T rows when the caller stores it keys-contiguous.
//  * Softmax runs in the exp2 domain with fp32 statistics; the scale is
//    folded into one FMA per score, and the running max (with the O
//    rescale it implies) only moves when a tile's max exceeds it by 2^8.
//  * K/V tiles are buffer-loaded and double-buffered in LDS: one barrier
//    per key tile, the loads of tile j+1 in flight while tile j computes.
//  * Causal: tiles above an item's last query are skipped, only tiles that
//    cross the diagonal evaluate the mask.
//  * Schedule: stream-K (equal key-tile ranges over one resident wave of
//    workgroups, split items folded by attn_merge_kernel) when items are
//    few, else one workgroup per item, longest first.
// VALU paths (fp32 math, any element type): attn_fwd_split_kernel for
// head_dim in {8, 16, 32, 64, 128} (16 lanes per query row, key-split), and
// attn_fwd_generic_kernel (one thread per query row) for any other
// head_dim <= 256.
#include "common.h"
#include "lds_dma.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
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

constexpr int kAttnBN = 64;  // keys per tile of the bf16 kernel
// At head_dim 16 the O^T tile has 16 unused rows; row 24 of the V^T tile
// holds ones (no tile load writes rows past 21 there), so O^T row 24 -- the
// first lane half's register 12 -- is the row sum of the bf16 P.
constexpr int kAttnOnesRow = 24;

// Key tiles item wg walks: all of them, or (causal) up to its last query.
template <int NW>
__host__ __device__ __forceinline__ int attn_tiles(int wg, int S, int G, int ntasks, bool causal) {
  const int last_task = min(wg * NW + NW - 1, ntasks - 1);
  const int kend = causal ? min(S, (last_task / G) * 32 + 32) : S;
  return (kend + kAttnBN - 1) / kAttnBN;
}

// Item order.  Stream-K (alt): long and short items alternate (positions
// 0, 2, 4, .. take items nwg-1, nwg-2, ..; positions 1, 3, .. take items
// 0, 1, ..), so any contiguous run of tiles holds a similar number of item
// starts.  One item per workgroup (!alt): longest first, so the hardware
// dispatcher's greedy placement ends with the short items.
__host__ __device__ __forceinline__ int attn_pos_item(int p, int nwg, bool alt) {
  return (alt && (p & 1)) ? (p >> 1) : nwg - 1 - (alt ? (p >> 1) : p);
}

// Where tile v of the stream-K sequence lies.  The sequence walks positions
// p = 0.., and within a position the BH (batch, kv-head) pairs, each with
// the item's key tiles in order.  Wave-level: a lane-parallel prefix sum
// over positions; every output is wave-uniform.  Requires 0 <= v < total.
struct AttnLoc {
  int wg, bk, kb, nkb, start;  // item, pair, tile within item, item tiles, v of its tile 0
};
template <int NW>
__device__ __forceinline__ AttnLoc attn_locate(int v, int lane, int nwg, int BH, int S, int G,
                                               int ntasks, bool walk, bool alt) {
  const int per = (nwg + 63) / 64;
  int cnt = 0;
  for (int i = 0; i < per; ++i) {
    const int p = lane * per + i;
    if (p < nwg) cnt += attn_tiles<NW>(attn_pos_item(p, nwg, alt), S, G, ntasks, walk);
  }
  cnt *= BH;
  int incl = cnt;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  const int L = __ffsll(static_cast<unsigned long long>(__ballot(v < incl))) - 1;
  int base = __shfl(incl - cnt, L);
  int p = L * per, nt = 1;
  for (int i = 0; i < per; ++i, ++p) {
    nt = attn_tiles<NW>(attn_pos_item(p, nwg, alt), S, G, ntasks, walk);
    if (v < base + nt * BH) break;
    base += nt * BH;
  }
  AttnLoc r;
  r.wg = __builtin_amdgcn_readfirstlane(attn_pos_item(p, nwg, alt));
  r.nkb = __builtin_amdgcn_readfirstlane(nt);
  const int local = __builtin_amdgcn_readfirstlane(v - base);
  r.bk = local / r.nkb;
  r.kb = local - r.bk * r.nkb;
  r.start = __builtin_amdgcn_readfirstlane(base) + r.bk * r.nkb;
  return r;
}

// First tile of item w = p*BH + bk in the (!alt) sequence, and its length.
template <int NW>
__device__ __forceinline__ int2 attn_item_range(int w, int lane, int nwg, int BH, int S, int G,
                                                int ntasks, bool walk) {
  const int p = w / BH, bk = w - (w / BH) * BH;
  int part = 0;
  for (int i = lane; i < p; i += 64) part += attn_tiles<NW>(attn_pos_item(i, nwg, false), S, G, ntasks, walk);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off);
  const int nt = attn_tiles<NW>(attn_pos_item(p, nwg, false), S, G, ntasks, walk);
  const int start = __builtin_amdgcn_readfirstlane(part * BH + bk * nt);
  return make_int2(start, start + nt);
}

// First tile of workgroup w's range when T tiles are shared by P workgroups.
__host__ __device__ __forceinline__ int attn_range_begin(int w, int T, int P) {
  return static_cast<int>(static_cast<int64_t>(w) * T / P);
}


// Writes one query row of O (bf16) from the MFMA accumulator layout, with
// the softmax normaliser 1/l, and its log-sum-exp (m is in log2 units).
template <int HD>
__device__ __forceinline__ void attn_store_row(bf16* orow, const f32x16_t* acc, float m, float l,
                                               int hf, float* lse) {
  constexpr int DT = (HD + 31) / 32;
  const float inv = l > 0.f ? 1.f / l : 0.f;
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
  if (lse && hf == 0) *lse = l > 0.f ? (m + __log2f(l)) * kLn2 : -INFINITY;
}

// One 64-key tile for one wave (32 query rows of one head): S^T = K Q^T from
// the staged K rows kt (row pitch KROW), the mask (MASKED: keys past S,
// causality, the key mask kmrow of the batch row), the softmax update of
// (m_i, l_i, acc) and O^T += V^T P^T from the staged V^T rows vt (pitch
// VROW).  Lane (n, hf) owns query row qi; l_i is the lane's half of the row
// sum.  FIXED: Q was pre-scaled by scale * log2(e) and bounded, P = exp2 of
// the accumulator with no reference max.  RSM: the caller keeps a row of
// ones in the V^T tile's padding (row kAttnOnesRow), so the PV MFMAs also
// sum P into that row of O^T and the tile adds nothing to l_i.
template <int HD, bool CAUSAL, int MASK, bool FIXED, bool MASKED, int KROW, int VROW, bool RSM = false>
__device__ __forceinline__ void attn_tile(const uint16_t* kt, const uint16_t* vt, const bf16x8_t* qf,
                                          f32x16_t* acc, float& m_i, float& l_i, int key0, int qi,
                                          int S, int n, int hf, const uint8_t* kmrow, float scale_log2) {
  constexpr int BN = kAttnBN;
  constexpr int KSTEPS = HD / 16;
  constexpr int MT = BN / 32;
  constexpr int PS = BN / 16;
  constexpr int DT = (HD + 31) / 32;
  // Lazy rescaling: the running max used for exp2 only moves when a score
  // exceeds it by more than this (log2 units), so P stays <= 2^8.
  constexpr float kRescale = 8.f;
  f32x16_t st[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 16; ++r) st[mt][r] = 0.f;
  // The S MFMAs issue at raised wave priority: a wave that reaches them
  // keeps the matrix core fed ahead of the softmax VALU work of the other
  // waves on its SIMD (measured: -1% at C3, -1.5% at hd 16; raising the
  // softmax or the PV MFMAs instead made the kernel slower).
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint4 a = *reinterpret_cast<const uint4*>(&kt[(32 * mt + n) * KROW + 16 * s + 8 * hf]);
      st[mt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), qf[s], st[mt], 0, 0, 0);
    }
  __builtin_amdgcn_s_setprio(0);
  if constexpr (MASKED && MASK == 0) {
    // key = key0 + 4 hf + off with off = 32 mt + 8 (r / 4) + r % 4 a constant
    // per register: one compare against the lane's last visible key
    const int lim = (CAUSAL ? min(qi, S - 1) : S - 1) - key0 - 4 * hf;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int off = 32 * mt + 8 * (r >> 2) + (r & 3);
        st[mt][r] = off <= lim ? st[mt][r] : -INFINITY;
      }
  } else if constexpr (MASKED) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = key0 + 32 * mt + 8 * (r >> 2) + 4 * hf + (r & 3);
        bool ok = key < S;
        if (CAUSAL && MASK != 2) ok = ok && key <= qi;
        if (MASK != 0) {
          const bool keep = kmrow[min(key, S - 1)] != 0;
          ok = ok && (MASK == 1 ? keep : (key > qi || !keep));
        }
        st[mt][r] = ok ? st[mt][r] : -INFINITY;
      }
  }
  if constexpr (!FIXED) {
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[mt][r]);
    mx = halves_max(mx) * scale_log2;  // scaled row max of this tile
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
  }
  const float m_use = FIXED || m_i == -INFINITY ? 0.f : m_i;
  // P in bf16, and its row sum from the same rounded values (v_dot2 with
  // (1, 1)), so the normalisation uses exactly the P of the PV product.
  uint4 pk[PS];
  float rs = 0.f;
#pragma unroll
  for (int s2 = 0; s2 < PS; ++s2) {
    const int mt = s2 >> 1, rb = 8 * (s2 & 1);
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      p[e] = FIXED ? __builtin_amdgcn_exp2f(st[mt][rb + e])
                   : __builtin_amdgcn_exp2f(fmaf(st[mt][rb + e], scale_log2, -m_use));
    pk[s2].x = pack2<bf16>(p[0], p[1]);
    pk[s2].y = pack2<bf16>(p[2], p[3]);
    pk[s2].z = pack2<bf16>(p[4], p[5]);
    pk[s2].w = pack2<bf16>(p[6], p[7]);
    if constexpr (!RSM) {
      rs = dot2_bf16(pk[s2].x, kOnesBf16x2, rs);
      rs = dot2_bf16(pk[s2].y, kOnesBf16x2, rs);
      rs = dot2_bf16(pk[s2].z, kOnesBf16x2, rs);
      rs = dot2_bf16(pk[s2].w, kOnesBf16x2, rs);
    }
  }
  if constexpr (!RSM) l_i += rs;
  // O^T += V^T P^T over PS k-steps of 16 keys.
#pragma unroll
  for (int s2 = 0; s2 < PS; ++s2) {
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
}

// LDS tile sizes of attn_fwd_mfma_body / attn_fwd_kp_body (elements).
template <int HD, bool VT>
struct AttnLds {
  static constexpr int DT = (HD + 31) / 32;
  static constexpr int KSL = HD / 8 + 1;
  static constexpr int KBUF = kAttnBN * 8 * KSL;
  static constexpr int VSL = kAttnBN / 8 + 1;
  static constexpr int VROW = VT ? 8 * VSL : kAttnBN + 4;
  static constexpr int VINS = (HD * VSL + 63) / 64;
  static constexpr int VBUF = (VT && VINS * 512 > DT * 32 * VROW) ? VINS * 512 : DT * 32 * VROW;
};

// Whether the fixed-reference path applies, from the QK-norm temperature on
// the device: |q.k| <= 1.03 |temperature| (q unit norm, k of norm
// |temperature|, with room for the bf16 roundings), and the path needs that
// bound times scale * log2(e) to be <= 48 (log2 units).  Read by every lane
// from one address and made wave-uniform.
__device__ __forceinline__ bool attn_fixed_from_temperature(const void* tau, int tau_bf16,
                                                            float scale_log2) {
  float t;
  if (tau_bf16) {
    t = __uint_as_float(static_cast<uint32_t>(*static_cast<const uint16_t*>(tau)) << 16);
  } else {
    t = *static_cast<const float*>(tau);
  }
  t = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(t)));
  return 1.03f * fabsf(t) * scale_log2 <= 48.f;
}

template <int HD, bool CAUSAL, int MASK, bool VT, int NW, bool FIXED>
__device__ __forceinline__ void attn_fwd_mfma_body(
    uint16_t* __restrict__ Ks, uint16_t* __restrict__ Vt, const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    bf16* __restrict__ o, float* __restrict__ lse, const uint8_t* __restrict__ kmask,
    int S, int Hq, int Hkv, int G, int ntasks, int nwg, int BH, int T, int per_item,
    float* __restrict__ ws, int4* __restrict__ desc,
    int64_t qs0, int64_t qs1, int64_t qs2,
    int64_t ks0, int64_t ks1, int64_t ks2,
    int64_t vs0, int64_t vs1, int64_t vs2,
    int64_t os0, int64_t os1, int64_t os2, float scale_log2) {
  // VT: V is stored transposed ([.., hd, S], keys contiguous, row stride
  // vs2 between d rows) and is staged with plain 16-byte copies; otherwise
  // V is [.., S, hd] and is transposed while staged.
  constexpr int BN = kAttnBN;           // keys per tile
  constexpr int KSTEPS = HD / 16;       // k-steps of S^T = K Q^T
  constexpr int DT = (HD + 31) / 32;    // 32-row d tiles of O^T
  // LDS rows are padded by one 16-byte slot (8 elements) so that the MFMA
  // operand reads of 16 consecutive rows hit distinct banks.  K (and V^T
  // when V comes keys-contiguous) is loaded straight into LDS: a wave's
  // buffer load writes 64 consecutive slots, one per lane, and the lanes
  // that land on a pad slot load nothing (an offset past num_records).
  constexpr int DC = HD / 8;            // 16-byte chunks per K/V row
  constexpr int KSL = DC + 1;           // LDS slots per K row
  constexpr int KROW = 8 * KSL;         // padded LDS row of K (elements)
  constexpr int VSL = BN / 8 + 1;       // LDS slots per V^T row (direct path)
  constexpr int VROW = VT ? 8 * VSL : BN + 4;  // padded LDS row of V^T (elements)
  constexpr int NT = 64 * NW;                       // threads per workgroup
  constexpr int VCH = ((BN / 2) * DC + NT - 1) / NT;  // V key-pair units per thread
  constexpr int VINS = (HD * VSL + 63) / 64;        // V^T load instructions per tile
  constexpr int KBUF = BN * KROW;                   // BN * KSL slots
  constexpr int KINS = BN * KSL / 64;               // K load instructions per tile
  constexpr int VBUF = (VT && VINS * 512 > DT * 32 * VROW) ? VINS * 512 : DT * 32 * VROW;
  // FIXED: the caller bounds |q.k| by beta with beta * scale <= 48 in log2
  // units, so exp2 of a scaled score lies in [2^-48, 2^48] and needs no
  // reference max at all (P, l and O stay far inside the bf16 / fp32 range):
  // Q is scaled by scale * log2(e) as it is loaded, P = exp2 of the MFMA
  // accumulator with no FMA, and there is no per-tile max or rescaling.  The
  // scaled Q is rounded to bf16 once (2^-9 relative per element, the size of
  // Q's own bf16 rounding).
  constexpr bool fixed_max = FIXED;
  static_assert(KBUF == AttnLds<HD, VT>::KBUF && VBUF == AttnLds<HD, VT>::VBUF,
                "LDS sizes agree with the kernel's arrays");

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n = lane & 31, hf = lane >> 5;
  // Stream-K schedule: the grid is one resident wave of workgroups, and
  // workgroup w takes tiles [T*w/P, T*(w+1)/P) of the sequence of all
  // (item, key tile) pairs, so every workgroup gets the same number of key
  // tiles however uneven the causal items are.  An item that lies whole in
  // the range is written out directly; a piece of one (a chunk) stores its
  // (m, l, unnormalised O) in partial slot 2w (the range's first chunk) or
  // 2w+1 (its last), for attn_merge_kernel.  The workgroup whose range holds
  // tile 0 of a split item records it in desc[w]; desc[w].y = 0 otherwise.
  // With per_item set, the grid has one workgroup per item instead (longest
  // first) and nothing is split.
  const int P = gridDim.x;
  const bool walk = CAUSAL && MASK != 2;
  const bool alt = per_item == 0;
  int v_begin, v_end;
  if (alt) {
    v_begin = attn_range_begin(blockIdx.x, T, P);
    v_end = attn_range_begin(blockIdx.x + 1, T, P);
  } else {
    const int2 r = attn_item_range<NW>(blockIdx.x, lane, nwg, BH, S, G, ntasks, walk);
    v_begin = r.x;
    v_end = r.y;
  }

  // HD 16: P's row sums come from the PV MFMAs (a row of ones in V^T)
  constexpr bool RSM = HD == 16;
  static_assert(!RSM || (VINS * 64 <= kAttnOnesRow * VSL && kAttnOnesRow < DT * 32),
                "no V^T tile load reaches the row of ones");
  if (DT * 32 > HD) {  // zero the padding rows of both V^T buffers once (ones in the sum row)
    for (int i = tid; i < (DT * 32 - HD) * VROW; i += NT) {
      const uint16_t f = RSM && HD + i / VROW == kAttnOnesRow ? 0x3f80 : 0;
      Vt[HD * VROW + i] = f;
      Vt[VBUF + HD * VROW + i] = f;
    }
  }

  // Global loads go through buffer descriptors: each thread's byte offsets
  // within a tile are fixed (computed once, 32-bit), and a tile only moves
  // the descriptor base, in scalar registers.  num_records ends at the last
  // valid K (or row-major V) row, so rows at or past S read as zero with no
  // per-row test.
  constexpr int kRsrcFlags = 0x00020000;  // raw (untyped) access, gfx9 family
  constexpr uint32_t kOob = 0x80000000u;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  // With V^T rows (VT), K and V^T go straight to LDS: instruction j (of
  // KINS) fills K slots [64j, 64j+64); wave w issues j = w, w+NW, ..  With
  // row-major V, whose transpose needs registers anyway, K is staged through
  // registers too (KCH 16-byte chunks per thread): that variant stays under
  // the register budget of three waves per SIMD.
  constexpr int KIPW = VT ? (KINS + NW - 1) / NW : 1;
  constexpr int KCH = VT ? 1 : (BN * DC + NT - 1) / NT;
  uint32_t koffs[VT ? KIPW : KCH];
#pragma unroll
  for (int i = 0; i < (VT ? KIPW : KCH); ++i) {
    if constexpr (VT) {
      const int j = wv + NW * i, P = 64 * j + lane;
      const int r = P / KSL, c = P - r * KSL;
      koffs[i] = (j < KINS && c < DC) ? static_cast<uint32_t>((r * ks2 + c * 8) * 2) : kOob;
    } else {
      const int c = tid + NT * i;
      const int key = c / DC, dc = c - key * DC;
      koffs[i] = c < BN * DC ? static_cast<uint32_t>((key * ks2 + dc * 8) * 2) : kOob;
    }
  }
  // V^T rows (direct path): slot P <-> (d = P / VSL, 8-key chunk P % VSL)
  constexpr int VIPW = VT ? (VINS + NW - 1) / NW : 1;
  uint32_t vtoffs[VIPW];
#pragma unroll
  for (int i = 0; i < VIPW; ++i) {
    const int j = wv + NW * i, P = 64 * j + lane;
    const int d = P / VSL, c = P - d * VSL;
    vtoffs[i] = (VT && j < VINS && d < HD && c < BN / 8) ? static_cast<uint32_t>((d * vs2 + 8 * c) * 2) : kOob;
  }
  // row-major V: transposed through registers while staged
  uint32_t voff[VT ? 1 : VCH];
  if constexpr (!VT) {
#pragma unroll
    for (int j = 0; j < VCH; ++j) {
      const int c = tid + NT * j;
      const int kp = c / DC, dc = c - kp * DC;
      voff[j] = c < (BN / 2) * DC ? static_cast<uint32_t>((2 * kp * vs2 + dc * 8) * 2) : kOob;
    }
  }
  const uint32_t vrow_bytes = static_cast<uint32_t>(vs2 * 2);
  const uint32_t ks_lds = lds_addr(Ks), vt_lds = lds_addr(Vt);

  bool started = false;
  int chunk_no = 0;
  for (int vcur = v_begin; vcur < v_end; ++chunk_no) {
    const AttnLoc loc = attn_locate<NW>(vcur, lane, nwg, BH, S, G, ntasks, walk, alt);
    const int wg = loc.wg, bk = loc.bk, nkb = loc.nkb;
    const int kb0 = loc.kb, kb1 = min(nkb, kb0 + (v_end - vcur));
    vcur += kb1 - kb0;
    const int b = bk / Hkv, kvh = bk - b * Hkv;
    const int task = wg * NW + wave;
    const bool active = task < ntasks;
    const int qb = task / G;
    const int h = kvh * G + (task - qb * G);
    const int q0 = qb * 32;
    const int qi = q0 + n;
    const bf16* kbase = k + b * ks0 + kvh * ks1;
    const bf16* vbase = v + b * vs0 + kvh * vs1;

    // Q fragments (B operand of S^T = K Q^T): lane holds q[qi, 16s+8hf .. +7].
    bf16x8_t qf[KSTEPS];
    {
      const bf16* qrow = q + b * qs0 + h * qs1 + static_cast<int64_t>(qi) * qs2;
  #pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        uint4 raw = make_uint4(0, 0, 0, 0);
        if (active && qi < S) raw = *reinterpret_cast<const uint4*>(qrow + 16 * s + 8 * hf);
        if constexpr (fixed_max) {
          uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            w[e] = pack2<bf16>(__uint_as_float(w[e] << 16) * scale_log2,
                               __uint_as_float(w[e] & 0xffff0000u) * scale_log2);
          raw = make_uint4(w[0], w[1], w[2], w[3]);
        }
        qf[s] = as_bf16x8(raw);
      }
    }

    // Retire the Q loads here: otherwise the in-order vmcnt makes the first
    // MFMA of every iteration wait for the next tile's prefetch as well.
    __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)

    uint4 vreg[VT ? 1 : VCH][2];
    uint4 kreg[VT ? 1 : KCH];
    // Issue the loads of the tile at key0 into LDS buffer buf (K, and V^T
    // on the direct path) or registers (row-major V).
    auto fetch_tile = [&](int key0, int buf) {
      const int rows = min(BN, S - key0);  // valid keys in this tile (>= 1)
      const bf16* kt0 = kbase + static_cast<int64_t>(key0) * ks2;
      const int krec = static_cast<int>((rows - 1) * ks2 * 2 + HD * 2);
      if constexpr (VT) {
        const i32x4_t kr = raw_rsrc(kt0, krec);
#pragma unroll
        for (int i = 0; i < KIPW; ++i) {
          const int j = wv + NW * i;
          if (j < KINS) load16_to_lds(kr, ks_lds + (buf * KBUF + 512 * j) * 2, koffs[i]);
        }
      } else {
        const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(kt0), 0, krec, kRsrcFlags);
#pragma unroll
        for (int i = 0; i < KCH; ++i)
          kreg[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(kr, koffs[i], 0, 0));
      }
      if constexpr (VT) {
        // Keys past S inside a d row are in memory (the next row's keys, or
        // the row padding): zero_tail() clears them in LDS.  num_records
        // stops the last row at S.
        const i32x4_t vr = raw_rsrc(vbase + key0, static_cast<int>((HD - 1) * vs2 * 2 + rows * 2));
#pragma unroll
        for (int i = 0; i < VIPW; ++i) {
          const int j = wv + NW * i;
          if (j < VINS)
            load16_to_lds(vr, vt_lds + (buf * VBUF + 512 * j) * 2, vtoffs[i]);
        }
      } else {
        const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<bf16*>(vbase + static_cast<int64_t>(key0) * vs2), 0,
            static_cast<int>((rows - 1) * vs2 * 2 + HD * 2), kRsrcFlags);
#pragma unroll
        for (int j = 0; j < VCH; ++j) {
          vreg[j][0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, voff[j], 0, 0));
          vreg[j][1] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(vr, voff[j] + vrow_bytes, 0, 0));
        }
      }
    };
    // Row-major V: K rows and the transposed V from registers into buffer buf.
    auto stage = [&](int buf) {
      if constexpr (!VT) {
        uint16_t* kd = Ks + buf * KBUF;
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
          const int c = tid + NT * i;
          const int key = c / DC, dc = c - key * DC;
          if ((BN * DC) % NT == 0 || c < BN * DC) *reinterpret_cast<uint4*>(&kd[key * KROW + dc * 8]) = kreg[i];
        }
        uint16_t* vd = Vt + buf * VBUF;
#pragma unroll
        for (int j = 0; j < VCH; ++j) {
          const int u = tid + NT * j;
          const int kp = u / DC, dc = u - kp * DC;
          if (((BN / 2) * DC) % NT == 0 || u < (BN / 2) * DC) {
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
    // Wait for this wave's loads (LDS writes included), then for every wave.
    auto land = [&]() {
      __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0)
      __syncthreads();
    };
    // Direct V^T path, last tile of the sequence: zero the keys at or past S
    // (a uniform branch; S % 8 == 0 here).  Follows land(), ends with a barrier.
    auto zero_tail = [&](int key0, int buf) {
      if (VT && key0 + BN > S) {
        const int valid = S - key0, w = BN - valid;
        uint16_t* vd = Vt + buf * VBUF;
        for (int i = tid; i < HD * w; i += NT) {
          const int d = i / w;
          vd[d * VROW + valid + (i - d * w)] = 0;
        }
        __syncthreads();
      }
    };

    // l_i: this lane's part of the row sum (its half of the keys); the two
    // halves of the wave are added once, after the chunk's last tile.
    float m_i = fixed_max ? 0.f : -INFINITY, l_i = 0.f;
    f32x16_t acc[DT];
  #pragma unroll
    for (int dt = 0; dt < DT; ++dt)
  #pragma unroll
      for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;

    // One key tile.  MASKED is compile-time, so the tiles that are fully
    // visible to every wave of the workgroup run with no mask code at all.
    const uint8_t* kmrow = MASK != 0 ? kmask + static_cast<int64_t>(b) * S : nullptr;
    auto tile = [&](int kb, auto masked_tag) {
      constexpr bool MASKED = decltype(masked_tag)::value;
      const int buf = kb & 1;
      attn_tile<HD, CAUSAL, MASK, FIXED, MASKED, KROW, VROW, RSM>(Ks + buf * KBUF, Vt + buf * VBUF, qf, acc, m_i,
                                                                 l_i, kb * BN, qi, S, n, hf, kmrow, scale_log2);
    };


    // Tiles [0, nfull) are in bounds and at or below the diagonal of every
    // wave of the workgroup; the rest need the mask.
    const int wg_qmin = ((wg * NW) / G) * 32;
    int nfull = 0;
    if (MASK == 0) nfull = min(CAUSAL ? (wg_qmin + 1) / BN : nkb, S / BN);
    nfull = min(nfull, nkb);

    // This chunk's tiles [kb0, kb1): unmasked ones first, then masked.  The
    // barrier that ended the previous chunk's last tile lets both LDS
    // buffers be refilled.
    const int nf = max(kb0, min(nfull, kb1));
    fetch_tile(kb0 * BN, kb0 & 1);
    stage(kb0 & 1);
    land();
    zero_tail(kb0 * BN, kb0 & 1);
    // `active` is wave-uniform: branch on it rather than masking lanes.
    const bool wave_active = __builtin_amdgcn_readfirstlane(active ? 1 : 0) != 0;
    int kb = kb0;
    for (; kb < nf; ++kb) {
      // The next tile goes into the other buffer, which every wave finished
      // reading before the barrier that ended the previous iteration.
      if (kb + 1 < kb1) fetch_tile((kb + 1) * BN, (kb & 1) ^ 1);
      if (wave_active) tile(kb, std::false_type());
      if (kb + 1 < kb1) stage((kb & 1) ^ 1);
      land();
      if (kb + 1 < kb1) zero_tail((kb + 1) * BN, (kb & 1) ^ 1);
    }
    for (; kb < kb1; ++kb) {
      if (kb + 1 < kb1) fetch_tile((kb + 1) * BN, (kb & 1) ^ 1);
      const bool live = wave_active && !(CAUSAL && MASK != 2 && kb * BN > q0 + 31);
      if (live) tile(kb, std::true_type());
      if (kb + 1 < kb1) stage((kb & 1) ^ 1);
      land();
      if (kb + 1 < kb1) zero_tail((kb + 1) * BN, (kb & 1) ^ 1);
    }

    if constexpr (RSM) {
      // O^T row 24: register 12 of the lanes with hf = 0 (rescaled with O)
      if (wave_active) l_i = halves_sum(hf == 0 ? acc[0][12] : 0.f);
    } else {
      if (wave_active) l_i = halves_sum(l_i);
    }
    if (kb0 == 0 && kb1 == nkb) {
      if (wave_active && qi < S)
        attn_store_row<HD>(o + b * os0 + h * os1 + static_cast<int64_t>(qi) * os2, acc, m_i, l_i, hf,
                           lse ? lse + (static_cast<int64_t>(b) * Hq + h) * S + qi : nullptr);
    } else {
      // ws = [slot][wave][DT*4][64] partial O as 4 bf16 (uint2), then
      // [slot][wave][64] float2 (m, l), 2P slots.  O is relative to m and
      // bounded by l * max|v|, so bf16 keeps its range; the merge adds one
      // bf16 rounding (2^-9 relative) to the result.
      uint2* wacc = reinterpret_cast<uint2*>(ws);
      float2* wml = reinterpret_cast<float2*>(ws + static_cast<int64_t>(2 * P) * NW * 64 * DT * 8);
      const int slot = 2 * blockIdx.x + (chunk_no == 0 ? 0 : 1);
      const int64_t sw = static_cast<int64_t>(slot) * NW + wave;
      if (wave_active) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4)
            wacc[(sw * DT * 4 + dt * 4 + g4) * 64 + lane] =
                make_uint2(pack2<bf16>(acc[dt][4 * g4], acc[dt][4 * g4 + 1]),
                           pack2<bf16>(acc[dt][4 * g4 + 2], acc[dt][4 * g4 + 3]));
        wml[sw * 64 + lane] = make_float2(m_i, l_i);
      }
      if (kb0 == 0) {
        started = true;
        if (tid == 0) desc[blockIdx.x] = make_int4(loc.start, nkb, wg, bk);
      }
    }
  }
  if (!per_item && !started && tid == 0) desc[blockIdx.x] = make_int4(0, 0, 0, 0);
}

// FXM: 0 running row max, 1 fixed reference (the host has bounded |q.k|),
// 2 either, chosen per launch from the temperature on the device (no host
// read of it, and a captured graph follows later temperatures).
// With both paths in one kernel (FXM 2) the register budget is held to
// three waves per SIMD at HD <= 64, the occupancy each path has alone.
template <int HD, bool CAUSAL, int MASK, bool VT, int NW, int FXM>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu((FXM == 2 && HD <= 64) ? 3 : 1))) void attn_fwd_mfma_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    bf16* __restrict__ o, float* __restrict__ lse, const uint8_t* __restrict__ kmask,
    int S, int Hq, int Hkv, int G, int ntasks, int nwg, int BH, int T, int per_item,
    float* __restrict__ ws, int4* __restrict__ desc,
    int64_t qs0, int64_t qs1, int64_t qs2,
    int64_t ks0, int64_t ks1, int64_t ks2,
    int64_t vs0, int64_t vs1, int64_t vs2,
    int64_t os0, int64_t os1, int64_t os2, float scale_log2, const void* tau, int tau_bf16) {
  using Lds = AttnLds<HD, VT>;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2 * Lds::KBUF];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2 * Lds::VBUF];
#define HYDRA_MFMA_BODY(FX)                                                                  \
  attn_fwd_mfma_body<HD, CAUSAL, MASK, VT, NW, FX>(Ks, Vt, q, k, v, o, lse, kmask, S, Hq, Hkv, \
                                                   G, ntasks, nwg, BH, T, per_item, ws, desc, \
                                                   qs0, qs1, qs2, ks0, ks1, ks2, vs0, vs1,    \
                                                   vs2, os0, os1, os2, scale_log2)
  if constexpr (FXM == 2) {
    if (attn_fixed_from_temperature(tau, tau_bf16, scale_log2)) HYDRA_MFMA_BODY(true);
    else HYDRA_MFMA_BODY(false);
  } else {
    HYDRA_MFMA_BODY(FXM == 1);
  }
#undef HYDRA_MFMA_BODY
}

// Key-split workgroups (V^T rows only).  A workgroup of KP x NW waves takes
// one or two items -- NW tasks each, as in attn_fwd_mfma_kernel -- one after
// the other, and for each item its KP groups of NW waves walk the item's
// key tiles in turn (group g: tiles g, g + KP, ..), each group staging its
// own tiles in LDS, one barrier per step.  At the end of an item, groups
// 1..KP-1 leave (O, m, l) in LDS and group 0 folds them in group order and
// writes the rows.  Items are taken longest first in snake order over the
// P workgroups (workgroup w: items w and 2P-1-w), so with P = items / 2
// resident workgroups each gets a long and a short item and the causal
// triangle balances without chunk partials or a merge kernel.  The second
// item's first tiles and Q rows are fetched before the first item's fold,
// so their latency hides behind it, and no CU waits for a second launch.
// Strides are 32-bit here (the host checks they fit) to keep the two
// items' state within the scalar registers.
//
// LDS: every group's buffer 0 (K, V^T) in the first third of the array,
// buffer 1 in the second, and the fold's exchange over buffer 1 and the
// rest: an item's first tiles always land in buffer 0, which the fold
// leaves alone.
template <int HD, int NW, int KP>
struct KpLds {
  using L = AttnLds<HD, true>;
  static constexpr int DT = L::DT;
  static constexpr int TILE = L::KBUF + L::VBUF;     // one group's K and V^T buffer (elements)
  static constexpr int XF = DT * 16 + 2;             // exchanged floats per lane: O, m, l
  static constexpr int XCH = (KP - 1) * NW * 64 * XF * 2;  // exchange size in elements
  static constexpr int XOFF = KP * TILE;             // exchange start: the buffer-1 region
  // At hd 64 the output rows leave through a per-wave LDS tile (group 0's
  // NW waves x 32 rows x HD), outside the buffers and the exchange.
  static constexpr int SOFF = XOFF + (XCH > KP * TILE ? XCH : KP * TILE);
  static constexpr int SIZE = SOFF + (HD == 64 ? NW * 32 * HD : 0);
};

template <int HD, bool CAUSAL, int MASK, int NW, int KP, bool FIXED>
__device__ __forceinline__ void attn_fwd_kp_body(
    uint16_t* __restrict__ smem, const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    bf16* __restrict__ o, float* __restrict__ lse, const uint8_t* __restrict__ kmask,
    int S, int Hq, int Hkv, int G, int ntasks, int nwg, int BH, int P,
    int qs0, int qs1, int qs2, int ks0, int ks1, int ks2,
    int vs0, int vs1, int vs2, int os0, int os1, int os2, float scale_log2, bool o16) {
  constexpr int BN = kAttnBN;
  constexpr int KSTEPS = HD / 16;
  constexpr int DT = (HD + 31) / 32;
  constexpr int DC = HD / 8;             // 16-byte chunks per K row
  constexpr int KSL = DC + 1;            // LDS slots per K row (one pad slot)
  constexpr int KROW = 8 * KSL;
  constexpr int VSL = BN / 8 + 1;        // LDS slots per V^T row
  constexpr int VROW = 8 * VSL;
  constexpr int VINS = (HD * VSL + 63) / 64;
  constexpr int KBUF = BN * KROW;
  constexpr int KINS = BN * KSL / 64;
  constexpr int VBUF = VINS * 512 > DT * 32 * VROW ? VINS * 512 : DT * 32 * VROW;
  constexpr int KIPW = (KINS + NW - 1) / NW;
  constexpr int VIPW = (VINS + NW - 1) / NW;
  using Lay = KpLds<HD, NW, KP>;
  constexpr int TILE = Lay::TILE;
  constexpr int NT = 64 * NW * KP;
  constexpr int XF = Lay::XF;
  static_assert(KBUF == AttnLds<HD, true>::KBUF && VBUF == AttnLds<HD, true>::VBUF,
                "LDS sizes agree with the kernel's array");
  constexpr uint32_t kOob = 0x80000000u;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wv / NW, wq = wv - grp * NW;  // key group, task within the item
  const int n = lane & 31, hf = lane >> 5;
  const bool walk = CAUSAL && MASK != 2;
  const int nitems = nwg * BH;
  // group grp's buffer b: K at smem + (b * KP + grp) * TILE, V^T after it
  auto kbuf = [&](int b) { return smem + (b * KP + grp) * TILE; };
  auto vbuf = [&](int b) { return smem + (b * KP + grp) * TILE + KBUF; };

  if constexpr (DT * 32 > HD) {  // zero the padding rows of every V^T buffer once
    constexpr int PADE = (DT * 32 - HD) * VROW;
    for (int i = tid; i < KP * 2 * PADE; i += NT) {
      const int bu = i / PADE, r = i - bu * PADE;  // bu = buffer * KP + group
      smem[bu * TILE + KBUF + HD * VROW + r] = 0;
    }
  }
  // Per-lane byte offsets within a tile (fixed for the kernel): K slot
  // P = 64j + lane <-> (key row P / KSL, chunk P % KSL); V^T slot P <-> (d row
  // P / VSL, 8-key chunk P % VSL); pad slots and slots past the tile get an
  // offset past num_records and load zeros.
  uint32_t koffs[KIPW];
#pragma unroll
  for (int i = 0; i < KIPW; ++i) {
    const int j = wq + NW * i, Pp = 64 * j + lane;
    const int r = Pp / KSL, c = Pp - r * KSL;
    koffs[i] = (j < KINS && c < DC) ? static_cast<uint32_t>((r * ks2 + c * 8) * 2) : kOob;
  }
  uint32_t vtoffs[VIPW];
  int vtkey[VIPW];  // first key of the slot's chunk (BN for pad slots)
#pragma unroll
  for (int i = 0; i < VIPW; ++i) {
    const int j = wq + NW * i, Pp = 64 * j + lane;
    const int d = Pp / VSL, c = Pp - d * VSL;
    const bool ok = j < VINS && d < HD && c < BN / 8;
    vtoffs[i] = ok ? static_cast<uint32_t>((d * vs2 + 8 * c) * 2) : kOob;
    vtkey[i] = ok ? 8 * c : BN;
  }

  // One item: position pos in the longest-first order.
  struct Item {
    int wg, nkb, b, kvh, h, q0, qi;
    bool active;
    const bf16* kbase;
    const bf16* vbase;
  };
  auto locate = [&](int pos) {
    Item it;
    const int p = pos / BH, bk = pos - p * BH;
    it.wg = attn_pos_item(p, nwg, false);
    it.nkb = attn_tiles<NW>(it.wg, S, G, ntasks, walk);
    it.b = bk / Hkv;
    it.kvh = bk - it.b * Hkv;
    const int task = it.wg * NW + wq;
    it.active = task < ntasks;
    const int qb = task / G;
    it.h = it.kvh * G + (task - qb * G);
    it.q0 = qb * 32;
    it.qi = it.q0 + n;
    it.kbase = k + static_cast<int64_t>(it.b) * ks0 + static_cast<int64_t>(it.kvh) * ks1;
    it.vbase = v + static_cast<int64_t>(it.b) * vs0 + static_cast<int64_t>(it.kvh) * vs1;
    return it;
  };
  // snake order: round r takes position r*P + w (r even) or r*P + P-1-w
  auto pos_of = [&](int r) {
    return r * P + ((r & 1) ? P - 1 - static_cast<int>(blockIdx.x) : static_cast<int>(blockIdx.x));
  };

  // The group's loads of tile kb of item `it` into its buffer buf.  Keys at
  // or past S (last tile only; S % 8 == 0 on this path) load as zeros: K
  // rows through num_records, V^T chunks through the lane's offset.
  auto fetch = [&](const Item& it, int kb, int buf) {
    const int key0 = kb * BN;
    const int rows = min(BN, S - key0);
    const i32x4_t kr = raw_rsrc(it.kbase + static_cast<int64_t>(key0) * ks2,
                                static_cast<int>((rows - 1) * ks2 * 2 + HD * 2));
    const uint32_t ks_lds = lds_addr(kbuf(buf));
    const uint32_t vt_lds = lds_addr(vbuf(buf));
#pragma unroll
    for (int i = 0; i < KIPW; ++i) {
      const int j = wq + NW * i;
      if (j < KINS) load16_to_lds(kr, ks_lds + 1024 * j, koffs[i]);
    }
    const i32x4_t vr = raw_rsrc(it.vbase + key0, static_cast<int>((HD - 1) * vs2 * 2 + rows * 2));
    if (key0 + BN <= S) {
#pragma unroll
      for (int i = 0; i < VIPW; ++i) {
        const int j = wq + NW * i;
        if (j < VINS) load16_to_lds(vr, vt_lds + 1024 * j, vtoffs[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < VIPW; ++i) {
        const int j = wq + NW * i;
        if (j < VINS) load16_to_lds(vr, vt_lds + 1024 * j, key0 + vtkey[i] < S ? vtoffs[i] : kOob);
      }
    }
  };
  auto land = [&]() {
    __builtin_amdgcn_s_waitcnt(0x3f70);  // vmcnt(0): this wave's loads, LDS writes included
    __syncthreads();
  };
  // Q fragments (B operand of S^T = K Q^T): lane holds q[qi, 16s+8hf .. +7],
  // loaded raw (no wait) and, once landed, FIXED: scaled by scale * log2(e)
  // and rounded to bf16 once.
  auto load_q = [&](const Item& it, uint4* raw) {
    const bf16* qrow = q + static_cast<int64_t>(it.b) * qs0 + static_cast<int64_t>(it.h) * qs1 +
                       static_cast<int64_t>(it.qi) * qs2;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      raw[s] = make_uint4(0, 0, 0, 0);
      if (it.active && it.qi < S) raw[s] = *reinterpret_cast<const uint4*>(qrow + 16 * s + 8 * hf);
    }
  };
  auto make_qf = [&](const uint4* raw, bf16x8_t* qf) {
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
      uint4 r = raw[s];
      if constexpr (FIXED) {
        uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = pack2<bf16>(__uint_as_float(w[e] << 16) * scale_log2,
                             __uint_as_float(w[e] & 0xffff0000u) * scale_log2);
        r = make_uint4(w[0], w[1], w[2], w[3]);
      }
      qf[s] = as_bf16x8(r);
    }
  };

  float* xch = reinterpret_cast<float*>(smem + Lay::XOFF);
  uint4 qraw[KSTEPS];
  // One item: its steps, then (when `nxt` is valid) the next item's first
  // tiles and Q rows, then the fold and the rows' stores.
  auto run_item = [&](const Item& cur, int nxt_pos) {
    bf16x8_t qf[KSTEPS];
    make_qf(qraw, qf);
    float m_i = FIXED ? 0.f : -INFINITY, l_i = 0.f;
    f32x16_t acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;

    // Tiles [0, nfull) are in bounds and at or below the diagonal of every
    // wave; the rest need the mask.
    const int nkb = cur.nkb;
    const int wg_qmin = ((cur.wg * NW) / G) * 32;
    int nfull = 0;
    if (MASK == 0) nfull = min(CAUSAL ? (wg_qmin + 1) / BN : nkb, S / BN);
    nfull = min(nfull, nkb);
    const uint8_t* kmrow = MASK != 0 ? kmask + static_cast<int64_t>(cur.b) * S : nullptr;
    const int nsteps = (nkb + KP - 1) / KP;
    // Steps [0, st_full) have every group's tile unmasked; the rest (at most
    // a few at the end of a causal item) run the masked code for all tiles.
    // Two loops rather than a per-tile choice: a join of the two tile codes
    // costs a copy of the accumulators every step.
    const int st_full = nfull / KP;
    int st = 0;
    for (; st < st_full; ++st) {
      const int kb = st * KP + grp, buf = st & 1;
      // The group's next tile goes into its other buffer, which the group
      // finished reading before the barrier that ended the previous step.
      if (kb + KP < nkb) fetch(cur, kb + KP, buf ^ 1);
      if (cur.active)
        attn_tile<HD, CAUSAL, MASK, FIXED, false, KROW, VROW>(kbuf(buf), vbuf(buf), qf, acc, m_i, l_i,
                                                             kb * BN, cur.qi, S, n, hf, kmrow, scale_log2);
      land();
    }
    for (; st < nsteps; ++st) {
      const int kb = st * KP + grp, buf = st & 1;
      if (kb + KP < nkb) fetch(cur, kb + KP, buf ^ 1);
      if (cur.active && kb < nkb && !(walk && kb * BN > cur.q0 + 31))
        attn_tile<HD, CAUSAL, MASK, FIXED, true, KROW, VROW>(kbuf(buf), vbuf(buf), qf, acc, m_i, l_i,
                                                            kb * BN, cur.qi, S, n, hf, kmrow, scale_log2);
      land();
    }
    // Every read of this item's tiles ended at the last barrier: the next
    // item's first tiles go into buffer 0 and its Q rows into registers
    // while this item folds (the exchange lies outside buffer 0).
    if (nxt_pos < nitems) {
      const Item nxt = locate(nxt_pos);
      if (grp < nxt.nkb) fetch(nxt, grp, 0);
      load_q(nxt, qraw);
    }
    // Fold the groups.  The exchange holds, per (group, wave), 4*DT rows
    // of 64 lanes x 16 bytes (O) and one of 64 x 8 bytes (m, l): every LDS
    // instruction moves one contiguous 1 KB (or 512 B) row.
    l_i = halves_sum(l_i);
    if (grp > 0) {
      float* xw = xch + static_cast<int64_t>((grp - 1) * NW + wq) * 64 * XF;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *reinterpret_cast<float4*>(xw + ((dt * 4 + r4) * 64 + lane) * 4) =
              make_float4(acc[dt][4 * r4], acc[dt][4 * r4 + 1], acc[dt][4 * r4 + 2], acc[dt][4 * r4 + 3]);
      *reinterpret_cast<float2*>(xw + DT * 16 * 64 + 2 * lane) = make_float2(m_i, l_i);
    }
    __syncthreads();
    const bool store = grp == 0 && cur.active && cur.qi < S;
    if (store) {
#pragma unroll
      for (int g = 1; g < KP; ++g) {
        const float* xw = xch + static_cast<int64_t>((g - 1) * NW + wq) * 64 * XF;
        const float2 ml = *reinterpret_cast<const float2*>(xw + DT * 16 * 64 + 2 * lane);
        const float m2 = ml.x, l2 = ml.y;
        float4 part[DT * 4];
#pragma unroll
        for (int j = 0; j < DT * 4; ++j) part[j] = *reinterpret_cast<const float4*>(xw + (j * 64 + lane) * 4);
        if constexpr (FIXED) {
          l_i += l2;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
              const float4 x = part[dt * 4 + r4];
              acc[dt][4 * r4] += x.x;
              acc[dt][4 * r4 + 1] += x.y;
              acc[dt][4 * r4 + 2] += x.z;
              acc[dt][4 * r4 + 3] += x.w;
            }
        } else if (m2 != -INFINITY) {  // a group that saw no key of this row adds nothing
          const float mn = fmaxf(m_i, m2);
          const float s1 = m_i == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_i - mn);
          const float s2 = __builtin_amdgcn_exp2f(m2 - mn);
          l_i = fmaf(l2, s2, l_i * s1);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
              const float4 x = part[dt * 4 + r4];
              acc[dt][4 * r4] = fmaf(x.x, s2, acc[dt][4 * r4] * s1);
              acc[dt][4 * r4 + 1] = fmaf(x.y, s2, acc[dt][4 * r4 + 1] * s1);
              acc[dt][4 * r4 + 2] = fmaf(x.z, s2, acc[dt][4 * r4 + 2] * s1);
              acc[dt][4 * r4 + 3] = fmaf(x.w, s2, acc[dt][4 * r4 + 3] * s1);
            }
          m_i = mn;
        }
      }
    }
    // Before the next item: its tiles and Q rows have landed, and group 0
    // has read the exchange before any group writes buffer 1 again.  The
    // rows are stored after that barrier, so the stores overlap the next
    // item's first step instead of holding the barrier.
    if (nxt_pos < nitems) land();
    bool staged = false;
    if constexpr (HD == 64) staged = o16;
    if (staged) {
      // The wave's 32 rows go to its LDS tile (16-byte chunks XOR-swizzled
      // by row, so the column writes of 32 rows spread over the banks) and
      // come back row-contiguous: each store instruction then writes 8
      // whole 128-byte rows, instead of 8-byte pieces of 32 rows (o16: the
      // host found the rows 16-byte aligned; otherwise the 8-byte stores).
      if (grp == 0 && cur.active) {
        uint16_t* sw = smem + Lay::SOFF + wq * 32 * HD;
        const float inv = l_i > 0.f ? 1.f / l_i : 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const int ch = 4 * dt + g4;
            uint2 w;
            w.x = pack2<bf16>(acc[dt][4 * g4 + 0] * inv, acc[dt][4 * g4 + 1] * inv);
            w.y = pack2<bf16>(acc[dt][4 * g4 + 2] * inv, acc[dt][4 * g4 + 3] * inv);
            *reinterpret_cast<uint2*>(sw + n * HD + ((ch ^ (n & 7)) << 3) + 4 * hf) = w;
          }
        if (lse && hf == 0 && cur.qi < S)
          lse[(static_cast<int64_t>(cur.b) * Hq + cur.h) * S + cur.qi] =
              l_i > 0.f ? (m_i + __log2f(l_i)) * kLn2 : -INFINITY;
        bf16* ob = o + static_cast<int64_t>(cur.b) * os0 + static_cast<int64_t>(cur.h) * os1;
        const int c = lane & 7;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 8 * i + (lane >> 3);
          const uint4 val = *reinterpret_cast<const uint4*>(sw + r * HD + ((c ^ (r & 7)) << 3));
          if (cur.q0 + r < S) *reinterpret_cast<uint4*>(ob + static_cast<int64_t>(cur.q0 + r) * os2 + 8 * c) = val;
        }
      }
    } else if (store) {
      attn_store_row<HD>(o + static_cast<int64_t>(cur.b) * os0 + static_cast<int64_t>(cur.h) * os1 +
                             static_cast<int64_t>(cur.qi) * os2, acc, m_i, l_i, hf,
                         lse ? lse + (static_cast<int64_t>(cur.b) * Hq + cur.h) * S + cur.qi : nullptr);
    }
  };

  // At most two items per workgroup (the launch makes P >= items / 2): the
  // body is written out twice rather than looped, which keeps the step
  // loop's register pressure at one item's.
  const int pos0 = pos_of(0);
  if (pos0 >= nitems) return;
  const int pos1 = pos_of(1);
  {
    const Item first = locate(pos0);
    if (grp < first.nkb) fetch(first, grp, 0);
    load_q(first, qraw);
    land();
    run_item(first, pos1);
  }
  if (pos1 >= nitems) return;
  run_item(locate(pos1), nitems);
}

template <int HD, bool CAUSAL, int MASK, int NW, int KP, int FXM>
__global__ __launch_bounds__(64 * NW * KP) void attn_fwd_kp_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    bf16* __restrict__ o, float* __restrict__ lse, const uint8_t* __restrict__ kmask,
    int S, int Hq, int Hkv, int G, int ntasks, int nwg, int BH, int P,
    int qs0, int qs1, int qs2, int ks0, int ks1, int ks2,
    int vs0, int vs1, int vs2, int os0, int os1, int os2, float scale_log2, const void* tau, int tau_bf16,
    int o16, unsigned long long* __restrict__ clk) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[KpLds<HD, NW, KP>::SIZE];
  // Clock stamps (measurement aid, off unless the host installed a buffer):
  // thread 0 records the shader-clock and wall-clock counters when the
  // workgroup starts and after its last rows are stored.
  unsigned long long t0 = 0, r0 = 0;
  if (clk) {
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
#define HYDRA_KP_BODY(FX)                                                                       \
  attn_fwd_kp_body<HD, CAUSAL, MASK, NW, KP, FX>(smem, q, k, v, o, lse, kmask, S, Hq, Hkv, G,    \
                                                 ntasks, nwg, BH, P, qs0, qs1, qs2, ks0, ks1, ks2, \
                                                 vs0, vs1, vs2, os0, os1, os2, scale_log2, o16 != 0)
  if constexpr (FXM == 2) {
    if (attn_fixed_from_temperature(tau, tau_bf16, scale_log2)) HYDRA_KP_BODY(true);
    else HYDRA_KP_BODY(false);
  } else {
    HYDRA_KP_BODY(FXM == 1);
  }
#undef HYDRA_KP_BODY
  if (clk && threadIdx.x == 0) {
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    unsigned long long* c = clk + 4 * static_cast<int64_t>(blockIdx.x);
    c[0] = t0;
    c[1] = t1;
    c[2] = r0;
    c[3] = r1;
  }
}

// Combines the chunks of split items.  One thread per (w, wave, lane),
// where w is the workgroup whose range holds the item's tile 0: lane l of a
// wave holds query l%32 and, for f = 0..DT*4-1, d = 32(f/4) + 8(f%4) +
// 4(l/32) + 0..3 -- the MFMA accumulator layout the partials were stored
// in.  The item's chunks are, in key order: workgroup w's last chunk (slot
// 2w+1, or 2w if the item starts w's range), then the first chunk (slot
// 2w') of each following workgroup w' whose range starts inside the item.
// They are folded in that order (online max), so the result is
// deterministic; the loads of up to four chunks are issued together.
template <int HD, int NW>
__global__ __launch_bounds__(256) void attn_merge_kernel(
    const float* __restrict__ ws, const int4* __restrict__ desc, bf16* __restrict__ o,
    float* __restrict__ lse, int P, int T, int S, int Hq, int Hkv, int G, int ntasks,
    int64_t os0, int64_t os1, int64_t os2) {
  constexpr int DT = (HD + 31) / 32;
  constexpr int F = DT * 4;  // 4-element groups per lane
  const int gid = blockIdx.x * 256 + threadIdx.x;
  const int lane = gid & 63;
  const int wave = (gid >> 6) % NW;
  const int w = gid / (64 * NW);
  if (w >= P) return;
  const int4 d = desc[w];
  // one 16-byte load: keep the compiler from splitting it across the exits
  asm volatile("" ::"v"(d.x), "v"(d.y), "v"(d.z), "v"(d.w));
  const int v_s = d.x, nkb = d.y, wg = d.z, bk = d.w;
  if (nkb == 0) return;
  const int task = wg * NW + wave;
  if (task >= ntasks) return;
  const int qb = task / G;
  const int b = bk / Hkv, kvh = bk - b * Hkv;
  const int h = kvh * G + (task - qb * G);
  const int qi = qb * 32 + (lane & 31), hf = lane >> 5;
  if (qi >= S) return;
  const uint2* wacc = reinterpret_cast<const uint2*>(ws);
  const float2* wml = reinterpret_cast<const float2*>(ws + static_cast<int64_t>(2 * P) * NW * 64 * DT * 8);
  // Range starts floor(w'T/P) compared without a division:
  // floor(w'T/P) < x  <=>  w'T < xP.
  const int64_t vend_p = static_cast<int64_t>(v_s + nkb) * P;
  int nc = 1;
  while (w + nc < P && static_cast<int64_t>(w + nc) * T < vend_p) ++nc;
  // the item opens w's range iff floor(wT/P) >= v_s (it cannot start before)
  const int slot0 = static_cast<int64_t>(w) * T >= static_cast<int64_t>(v_s) * P ? 2 * w : 2 * w + 1;
  float M = -INFINITY, L = 0.f;
  float acc[F][4];
#pragma unroll
  for (int g = 0; g < F; ++g) acc[g][0] = acc[g][1] = acc[g][2] = acc[g][3] = 0.f;
  for (int j0 = 0; j0 < nc; j0 += 4) {
    float2 ml[4];
    uint2 a[4][F];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + u;
      const int64_t sj = static_cast<int64_t>(j == 0 ? slot0 : 2 * (w + j)) * NW + wave;
      ml[u] = j < nc ? wml[sj * 64 + lane] : make_float2(-INFINITY, 0.f);
#pragma unroll
      for (int g = 0; g < F; ++g) a[u][g] = j < nc ? wacc[(sj * F + g) * 64 + lane] : make_uint2(0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      // a chunk in which this row saw no key has m = -inf, l = 0, O = 0
      if (ml[u].x == -INFINITY) continue;
      const float mn = fmaxf(M, ml[u].x);
      const float s_old = M == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(M - mn);
      const float s_new = __builtin_amdgcn_exp2f(ml[u].x - mn);
      M = mn;
      L = fmaf(s_new, ml[u].y, L * s_old);
#pragma unroll
      for (int g = 0; g < F; ++g) {
        acc[g][0] = fmaf(s_new, __uint_as_float(a[u][g].x << 16), acc[g][0] * s_old);
        acc[g][1] = fmaf(s_new, __uint_as_float(a[u][g].x & 0xffff0000u), acc[g][1] * s_old);
        acc[g][2] = fmaf(s_new, __uint_as_float(a[u][g].y << 16), acc[g][2] * s_old);
        acc[g][3] = fmaf(s_new, __uint_as_float(a[u][g].y & 0xffff0000u), acc[g][3] * s_old);
      }
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  bf16* orow = o + b * os0 + h * os1 + static_cast<int64_t>(qi) * os2;
#pragma unroll
  for (int g = 0; g < F; ++g) {
    const int dcol = 32 * (g >> 2) + 8 * (g & 3) + 4 * hf;
    if (dcol < HD) {
      uint2 w2;
      w2.x = pack2<bf16>(acc[g][0] * inv, acc[g][1] * inv);
      w2.y = pack2<bf16>(acc[g][2] * inv, acc[g][3] * inv);
      *reinterpret_cast<uint2*>(orow + dcol) = w2;
    }
  }
  if (lse && hf == 0)
    lse[(static_cast<int64_t>(b) * Hq + h) * S + qi] = L > 0.f ? (M + __log2f(L)) * kLn2 : -INFINITY;
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

// Clock-stamp buffer of the key-split kernel (hydra_attn_clock_stamps):
// 4 counters per workgroup, used by launches of at most g_clock_stamp_cap
// workgroups.  Host-side, process-wide; a measurement aid.
static unsigned long long* g_clock_stamps = nullptr;
static int64_t g_clock_stamp_cap = 0;

// With need != nullptr: only the plan -- *need = device scratch bytes the
// launch takes (stream-K partials and merge descriptors; 0 otherwise), no
// launch.  Otherwise the launch, with scratch from (ws, ws_bytes).
template <int HD>
static int launch_mfma(const void* q, const void* k, const void* v, void* o, float* lse,
                       const uint8_t* kmask, int mask_mode, int64_t B, int64_t Hq,
                       int64_t Hkv, int64_t S, const int64_t* qs, const int64_t* ks,
                       const int64_t* vs, const int64_t* os, bool causal, float scale,
                       float score_bound, const void* tau, int tau_bf16, void* ws_ptr,
                       size_t ws_bytes, size_t* need, hipStream_t st) {
  constexpr int NW = 4;  // waves per workgroup; GQA heads share each staged K/V tile
  constexpr int DT = (HD + 31) / 32;
  // V with unit stride along the keys is read as V^T rows (vs[3] apart).
  const bool vt = vs[2] == 1 && vs[3] != 1;
  const int G = static_cast<int>(Hq / Hkv);
  const int nqb = static_cast<int>((S + 31) / 32);
  const int ntasks = G * nqb;
  const int nwg = (ntasks + NW - 1) / NW;
  const int BH = static_cast<int>(B * Hkv);
  const int iS = static_cast<int>(S);
  // The reference-SDPA mask mode opens keys above the diagonal, so it walks
  // every key tile (no causal tile skipping).
  const bool walk = causal && mask_mode != HYDRA_MASK_REFERENCE_SDPA;
  int64_t T64 = 0;
  for (int w = 0; w < nwg; ++w) T64 += attn_tiles<NW>(w, iS, G, ntasks, walk);
  T64 *= BH;
  if (T64 >= (int64_t(1) << 31)) return fail(HYDRA_ERR_ARG, "attn_fwd: too many key tiles");
  const int T = static_cast<int>(T64);

  const float sl2 = scale * kLog2e;
  auto Q = static_cast<const bf16*>(q);
  auto K = static_cast<const bf16*>(k);
  auto V = static_cast<const bf16*>(v);
  auto O = static_cast<bf16*>(o);
  // A usable bound on |q.k| (and no key mask) selects the kernel without a
  // reference max; the bound on the scaled scores is in log2 units.
  const float m_fix = score_bound > 0.f ? score_bound * sl2 : INFINITY;
  const bool use_fixed = mask_mode == HYDRA_MASK_NONE && m_fix <= 48.f;
  auto go = [&](auto c_tag, auto m_tag, auto f_tag) -> int {
    constexpr bool C = decltype(c_tag)::value;
    constexpr int M = decltype(m_tag)::value;
    constexpr int FX = decltype(f_tag)::value;
    // Schedule.  With at least two items per resident workgroup slot, one
    // workgroup per item (longest first) lets the dispatcher balance the
    // load.  With fewer: for V^T rows, key-split workgroups (one item per
    // workgroup, its key tiles shared by KP groups of waves, no merge pass);
    // otherwise stream-K, one resident wave of workgroups, each with an
    // equal share of the key tiles, and a merge pass.  HYDRA_ATTN_SCHED=
    // streamk or kp forces the V^T choice; HYDRA_ATTN_WGS=n forces stream-K
    // on n workgroups, HYDRA_ATTN_WGS=0 one workgroup per item.
    // Resident slots from one instantiation per (causal, mask mode) --
    // without a key mask the one that picks its fixed-max path on the device
    // (FX 2), whichever runs: the workspace query sees no bound or
    // temperature, so the schedule it sizes for must not depend on them.
    constexpr int FXS = M == 0 ? 2 : 0;
    const int64_t slots = static_cast<int64_t>(device_cus()) *
                          blocks_per_cu(reinterpret_cast<const void*>(
                                            vt ? attn_fwd_mfma_kernel<HD, C, M, true, NW, FXS>
                                               : attn_fwd_mfma_kernel<HD, C, M, false, NW, FXS>),
                                        64 * NW);
    const int64_t items = static_cast<int64_t>(nwg) * BH;
    const char* sched = getenv("HYDRA_ATTN_SCHED");
    // the key-split kernel takes 32-bit strides
    auto fits32 = [](const int64_t* x, int n) {
      for (int i = 0; i < n; ++i)
        if (x[i] < 0 || x[i] > INT32_MAX) return false;
      return true;
    };
    const bool s32 = fits32(qs, 3) && fits32(ks, 3) && fits32(vs, 4) && fits32(os, 3);
    bool kp = vt && s32 && items < 2 * slots;
    if (sched && strcmp(sched, "streamk") == 0) kp = false;
    if (sched && strcmp(sched, "kp") == 0) kp = vt && s32;
    if (getenv("HYDRA_ATTN_WGS")) kp = false;
    if (kp) {
      if (need) {
        *need = 0;
        return HYDRA_OK;
      }
      constexpr int KP = HD == 128 ? 2 : 3;  // key groups (LDS: KP double-buffered K/V^T tiles)
      auto kkern = attn_fwd_kp_kernel<HD, C, M, NW, KP, FX>;
      // one resident wave of workgroups, each taking two items (more
      // workgroups when there are more than two items per resident slot)
      const int64_t kslots = static_cast<int64_t>(device_cus()) *
                             std::max(1, blocks_per_cu(reinterpret_cast<const void*>(kkern), 64 * NW * KP));
      const int Pk = static_cast<int>(std::min<int64_t>(items, std::max<int64_t>(kslots, (items + 1) / 2)));
      const int32_t qs32[3] = {(int32_t)qs[0], (int32_t)qs[1], (int32_t)qs[2]};
      const int32_t ks32[3] = {(int32_t)ks[0], (int32_t)ks[1], (int32_t)ks[2]};
      const int32_t vs32[3] = {(int32_t)vs[0], (int32_t)vs[1], (int32_t)vs[3]};
      const int32_t os32[3] = {(int32_t)os[0], (int32_t)os[1], (int32_t)os[2]};
      // 16-byte aligned output rows take whole-row stores through LDS (hd
      // 64); others the 8-byte stores (the workspace query cannot see the
      // pointer, so the choice does not change the schedule)
      const bool o16 = (reinterpret_cast<uintptr_t>(O) & 15) == 0 && os[0] % 8 == 0 && os[1] % 8 == 0 &&
                       os[2] % 8 == 0;
      kkern<<<dim3(static_cast<unsigned>(Pk)), 64 * NW * KP, 0, st>>>(
          Q, K, V, O, lse, kmask, iS, (int)Hq, (int)Hkv, G, ntasks, nwg, BH, Pk, qs32[0], qs32[1], qs32[2],
          ks32[0], ks32[1], ks32[2], vs32[0], vs32[1], vs32[2], os32[0], os32[1], os32[2], sl2, tau, tau_bf16,
          o16 ? 1 : 0, Pk <= g_clock_stamp_cap ? g_clock_stamps : nullptr);
      return check_launch("attn_fwd_kp_kernel");
    }
    auto kern = vt ? attn_fwd_mfma_kernel<HD, C, M, true, NW, FX> : attn_fwd_mfma_kernel<HD, C, M, false, NW, FX>;
    int64_t P64 = slots;
    bool per_item = items >= 2 * slots;
    if (const char* e = getenv("HYDRA_ATTN_WGS")) {
      const int64_t x = atoll(e);
      per_item = x == 0;
      if (x > 0) P64 = x;
    }
    if (per_item) P64 = items;
    const int P = static_cast<int>(std::min<int64_t>(P64, T));
    // Does any item straddle two ranges (then the merge kernel runs)?
    auto range_of = [&](int64_t t) { return ((t + 1) * P + T - 1) / T - 1; };
    bool split = false;
    int64_t vpos = 0;
    for (int p = 0; p < nwg && !split && !per_item; ++p) {
      const int nt = attn_tiles<NW>(attn_pos_item(p, nwg, true), iS, G, ntasks, walk);
      for (int bk = 0; bk < BH; ++bk, vpos += nt)
        if (range_of(vpos) != range_of(vpos + nt - 1)) {
          split = true;
          break;
        }
    }
    float* part = nullptr;
    int4* desc = nullptr;
    // stream-K: partial slots, then the merge descriptors (one workgroup
    // per item takes none)
    const size_t pb = per_item ? 0 : static_cast<size_t>(2 * P) * NW * 64 * (DT * 8 + 2) * sizeof(float);
    const size_t wb = per_item ? 0 : pb + static_cast<size_t>(P) * sizeof(int4);
    if (need) {
      *need = wb;
      return HYDRA_OK;
    }
    if (wb > 0) {
      if (ws_ptr == nullptr || ws_bytes < wb)
        return fail(HYDRA_ERR_ARG, "attn_fwd: workspace of " + std::to_string(wb) +
                                       " bytes required (hydra_attn_fwd_workspace)");
      part = static_cast<float*>(ws_ptr);
      desc = reinterpret_cast<int4*>(static_cast<char*>(ws_ptr) + pb);
    }
    kern<<<dim3(static_cast<unsigned>(P)), 64 * NW, 0, st>>>(
        Q, K, V, O, lse, kmask, iS, (int)Hq, (int)Hkv, G, ntasks, nwg, BH, T, per_item ? 1 : 0, part, desc,
        qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vt ? vs[3] : vs[2], os[0], os[1], os[2], sl2,
        tau, tau_bf16);
    const int rc1 = check_launch("attn_fwd_mfma_kernel");
    if (rc1 != HYDRA_OK || !split) return rc1;
    const int64_t threads = static_cast<int64_t>(P) * NW * 64;
    attn_merge_kernel<HD, NW><<<dim3(static_cast<unsigned>((threads + 255) / 256)), 256, 0, st>>>(
        part, desc, O, lse, P, T, iS, (int)Hq, (int)Hkv, G, ntasks, os[0], os[1], os[2]);
    return check_launch("attn_merge_kernel");
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  using M0 = std::integral_constant<int, 0>;
  using M1 = std::integral_constant<int, 1>;
  using M2 = std::integral_constant<int, 2>;
  // fixed-reference mode: 0 none, 1 from the host's bound, 2 from the
  // temperature on the device
  using X0 = std::integral_constant<int, 0>;
  using X1 = std::integral_constant<int, 1>;
  using X2 = std::integral_constant<int, 2>;
  if (mask_mode == HYDRA_MASK_REFERENCE_SDPA) return go(F_(), M2(), X0());
  if (causal && mask_mode == HYDRA_MASK_KEY_PADDING) return go(T_(), M1(), X0());
  if (mask_mode == HYDRA_MASK_KEY_PADDING) return go(F_(), M1(), X0());
  const bool dev = tau != nullptr;
  if (causal) return dev ? go(T_(), M0(), X2()) : use_fixed ? go(T_(), M0(), X1()) : go(T_(), M0(), X0());
  return dev ? go(F_(), M0(), X2()) : use_fixed ? go(F_(), M0(), X1()) : go(F_(), M0(), X0());
}

// ---------------------------------------------------------------------------
// Key-split VALU kernel (fp32 / fp16, and bf16 shapes the MFMA kernel does
// not take), head_dim a compile-time HD in {8, 16, 32, 64, 128}: a
// workgroup takes 16 consecutive query rows of one (batch, head) and stages
// 64-key tiles of K and V (fp32, rows padded by one word so the 16 keys a
// row's lanes read fall in distinct banks) in LDS; each row is split over 16
// lanes, lane l taking keys l, l+16, .. of every tile with its own online
// softmax (exp2 domain, one rescale per tile), and the 16 partial states are
// merged by shuffles at the end.  Same semantics as attn_fwd_generic_kernel
// (mask modes, lse), the rows spread over 16x the threads.
// ---------------------------------------------------------------------------
template <typename T, int HD>
__global__ __launch_bounds__(256) void attn_fwd_split_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    T* __restrict__ o, float* __restrict__ lse, const uint8_t* __restrict__ kmask,
    int B, int S, int Hq, int Hkv, int causal, int mask_mode,
    int64_t qs0, int64_t qs1, int64_t qs2, int64_t ks0, int64_t ks1, int64_t ks2,
    int64_t vs0, int64_t vs1, int64_t vs2, int64_t vs3, int64_t os0, int64_t os1, int64_t os2,
    float scale) {
  constexpr int KL = 16;            // lanes per query row
  constexpr int RW = 256 / KL;      // query rows per workgroup
  constexpr int TK = 64;            // keys per staged tile
  constexpr int KPT = TK / KL;      // keys per lane per tile
  constexpr int KP = HD + 1;        // padded LDS row (words)
  __shared__ float Ks[TK * KP], Vs[TK * KP];
  __shared__ int Vis[TK];           // key usable under the key mask (modes 1, 2)
  const int BH = B * Hq;
  const int nsb = (S + RW - 1) / RW;
  // longest rows first: blocks of the last query rows are dispatched first
  const int bh = blockIdx.x % BH;
  const int sb = nsb - 1 - static_cast<int>(blockIdx.x / BH);
  const int b = bh / Hq, h = bh - b * Hq;
  const int j = h / (Hq / Hkv);
  const int tid = threadIdx.x, row = tid / KL, kl = tid % KL;
  // Above head_dim 64 a row's lanes also split the head dimension: lane
  // pair (2i, 2i+1) takes keys i, i + KL/2, .. and the two halves of d, and
  // adds its partial dot products with one shuffle (the whole q row and
  // output accumulator per lane would not fit in registers).
  constexpr int DS = HD > 64 ? 2 : 1;   // d-slices per row
  constexpr int DH = HD / DS;           // dims per lane
  constexpr int KLK = KL / DS;          // key lanes per row
  const int dh = kl % DS, kln = kl / DS;
  const int s = sb * RW + row;
  const bool live = s < S;
  const float qscale = scale * kLog2e;
  float qv[DH], acc[DH];
  {
    const T* qr = q + b * qs0 + h * qs1 + static_cast<int64_t>(live ? s : 0) * qs2 + dh * DH;
#pragma unroll
    for (int d = 0; d < DH; ++d) {
      qv[d] = to_f32(qr[d]) * qscale;
      acc[d] = 0.f;
    }
  }
  float m = -INFINITY, l = 0.f;
  const bool walk = causal && mask_mode != HYDRA_MASK_REFERENCE_SDPA;
  const int kend = walk ? min(S, sb * RW + RW) : S;
  const T* kb = k + b * ks0 + j * ks1;
  const T* vb = v + b * vs0 + j * vs1;
  // Head dims up to 64: the next tile's K and V are loaded into registers
  // before this tile's arithmetic, so the loads' latency hides behind it
  // (one tile in flight; written to LDS after the next barrier).
  constexpr bool PF = HD <= 64;
  constexpr int PER = PF ? TK * HD / 256 : 1;  // elements per thread per tile
  static_assert(!PF || TK * HD % 256 == 0, "whole tile per pass");
  float kpre[PER], vpre[PER];
  auto prefetch = [&](int t0) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = tid + 256 * u;
      const int kk = i / HD, d = i - kk * HD;
      const int t = t0 + kk;
      const bool in = t < S;
      kpre[u] = in ? to_f32(kb[static_cast<int64_t>(t) * ks2 + d]) : 0.f;
      vpre[u] = in ? to_f32(vb[static_cast<int64_t>(t) * vs2 + d * vs3]) : 0.f;
    }
  };
  if constexpr (PF) prefetch(0);
  for (int t0 = 0; t0 < kend; t0 += TK) {
    __syncthreads();
    if constexpr (PF) {
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int i = tid + 256 * u;
        const int kk = i / HD, d = i - kk * HD;
        Ks[kk * KP + d] = kpre[u];
        Vs[kk * KP + d] = vpre[u];
      }
    } else {
      for (int i = tid; i < TK * HD; i += 256) {
        const int kk = i / HD, d = i - kk * HD;
        const int t = t0 + kk;
        const bool in = t < S;
        Ks[kk * KP + d] = in ? to_f32(kb[static_cast<int64_t>(t) * ks2 + d]) : 0.f;
        Vs[kk * KP + d] = in ? to_f32(vb[static_cast<int64_t>(t) * vs2 + d * vs3]) : 0.f;
      }
    }
    if (mask_mode != HYDRA_MASK_NONE && tid < TK) {
      const int t = t0 + tid;
      Vis[tid] = t < S ? (kmask[static_cast<int64_t>(b) * S + t] != 0) : 0;
    }
    __syncthreads();
    if constexpr (PF) {
      if (t0 + TK < kend) prefetch(t0 + TK);
    }
    float x[KPT * DS];
    float mt = m;
#pragma unroll
    for (int u = 0; u < KPT * DS; ++u) {
      const int kk = kln + KLK * u;
      const int t = t0 + kk;
      bool vis = live && t < S;
      if (mask_mode == HYDRA_MASK_REFERENCE_SDPA) vis = vis && (t > s || Vis[kk] == 0);
      else {
        if (causal) vis = vis && t <= s;
        if (mask_mode == HYDRA_MASK_KEY_PADDING) vis = vis && Vis[kk] != 0;
      }
      float dot = 0.f;
      const float* kr = Ks + kk * KP + dh * DH;
#pragma unroll
      for (int d = 0; d < DH; ++d) dot = fmaf(qv[d], kr[d], dot);
      if constexpr (DS == 2) dot += __shfl_xor(dot, 1, KL);
      x[u] = vis ? dot : -INFINITY;
      mt = fmaxf(mt, x[u]);
    }
    if (mt == -INFINITY) continue;  // nothing visible to this lane yet
    if (mt > m) {
      const float alpha = __builtin_amdgcn_exp2f(m - mt);  // m = -inf -> 0
      l *= alpha;
#pragma unroll
      for (int d = 0; d < DH; ++d) acc[d] *= alpha;
      m = mt;
    }
#pragma unroll
    for (int u = 0; u < KPT * DS; ++u) {
      const float pu = __builtin_amdgcn_exp2f(x[u] - m);  // -inf -> 0
      l += pu;
      const float* vr = Vs + (kln + KLK * u) * KP + dh * DH;
#pragma unroll
      for (int d = 0; d < DH; ++d) acc[d] = fmaf(pu, vr[d], acc[d]);
    }
  }
  // merge the key lanes of the row (lanes of one d-slice: offsets >= DS)
  float mg = m;
#pragma unroll
  for (int off = KL / 2; off >= DS; off >>= 1) mg = fmaxf(mg, __shfl_xor(mg, off, KL));
  const float f = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - mg);
  l *= f;
#pragma unroll
  for (int off = KL / 2; off >= DS; off >>= 1) l += __shfl_xor(l, off, KL);
#pragma unroll
  for (int d = 0; d < DH; ++d) {
    float a = acc[d] * f;
#pragma unroll
    for (int off = KL / 2; off >= DS; off >>= 1) a += __shfl_xor(a, off, KL);
    acc[d] = a;
  }
  if (!live) return;
  const float inv = l > 0.f ? 1.f / l : 0.f;
  T* orow = o + b * os0 + h * os1 + static_cast<int64_t>(s) * os2 + dh * DH;
#pragma unroll
  for (int d = 0; d < DH; ++d)
    if (d % KLK == kln) orow[d] = from_f32<T>(acc[d] * inv);
  if (lse && kl == 0)
    lse[(static_cast<int64_t>(b) * Hq + h) * S + s] = l > 0.f ? (mg + __log2f(l)) * kLn2 : -INFINITY;
}

template <typename T>
static int launch_split(const void* q, const void* k, const void* v, void* o, float* lse,
                        const uint8_t* kmask, int mask_mode, int64_t B, int64_t Hq, int64_t Hkv,
                        int64_t S, int64_t hd, const int64_t* qs, const int64_t* ks,
                        const int64_t* vs, const int64_t* os, bool causal, float scale,
                        hipStream_t st) {
  const int64_t nblk = B * Hq * ((S + 15) / 16);
  const dim3 grid(static_cast<unsigned>(nblk));
  auto Q = static_cast<const T*>(q);
  auto K = static_cast<const T*>(k);
  auto V = static_cast<const T*>(v);
  auto O = static_cast<T*>(o);
#define HYDRA_SPLIT_LAUNCH(HD)                                                              \
  attn_fwd_split_kernel<T, HD><<<grid, 256, 0, st>>>(                                       \
      Q, K, V, O, lse, kmask, (int)B, (int)S, (int)Hq, (int)Hkv, causal ? 1 : 0, mask_mode, \
      qs[0], qs[1], qs[2], ks[0], ks[1], ks[2], vs[0], vs[1], vs[2], vs[3], os[0], os[1],   \
      os[2], scale)
  switch (hd) {
    case 8: HYDRA_SPLIT_LAUNCH(8); break;
    case 16: HYDRA_SPLIT_LAUNCH(16); break;
    case 32: HYDRA_SPLIT_LAUNCH(32); break;
    case 64: HYDRA_SPLIT_LAUNCH(64); break;
    default: HYDRA_SPLIT_LAUNCH(128); break;
  }
#undef HYDRA_SPLIT_LAUNCH
  return check_launch("attn_fwd_split_kernel");
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

extern "C" int hydra_attn_clock_stamps(void* stamps, int64_t max_workgroups) {
  HYDRA_REQUIRE(max_workgroups >= 0, "attn_clock_stamps: negative capacity");
  HYDRA_REQUIRE(stamps != nullptr || max_workgroups == 0, "attn_clock_stamps: null buffer");
  HYDRA_REQUIRE(reinterpret_cast<uintptr_t>(stamps) % 8 == 0, "attn_clock_stamps: buffer must be 8-byte aligned");
  hydra::g_clock_stamps = static_cast<unsigned long long*>(stamps);
  hydra::g_clock_stamp_cap = stamps ? max_workgroups : 0;
  return HYDRA_OK;
}

// hydra_attn_fwd, or with need != nullptr the scratch bytes it would take
// (pointers not needed then; they are assumed 16-byte aligned, so the
// answer covers the MFMA path whenever the shapes allow it).
static int attn_fwd_impl(const void* q, const void* k, const void* v, void* o,
                         float* lse, const uint8_t* key_mask, int mask_mode,
                         int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t hd,
                         const int64_t* qs, const int64_t* ks, const int64_t* vs,
                         const int64_t* os, int causal, float scale,
                         float score_bound, const void* bound_temperature,
                         int bound_temperature_dtype, int dtype, void* workspace,
                         int64_t workspace_bytes, size_t* need, void* stream) {
  if (need) *need = 0;
  HYDRA_REQUIRE(B >= 0 && S >= 0 && Hq >= 1 && Hkv >= 1 && hd >= 1, "attn_fwd: bad size");
  HYDRA_REQUIRE(bound_temperature == nullptr || bound_temperature_dtype == HYDRA_BF16 ||
                    bound_temperature_dtype == HYDRA_F32,
                "attn_fwd: the bound temperature must be bf16 or fp32");
  HYDRA_REQUIRE(Hq % Hkv == 0, "attn_fwd: n_heads must be a multiple of n_kv_heads");
  HYDRA_REQUIRE(qs && ks && vs && os, "attn_fwd: null stride array");
  HYDRA_REQUIRE(qs[3] == 1 && ks[3] == 1 && os[3] == 1,
                "attn_fwd: q, k and o must have unit stride along head_dim");
  HYDRA_REQUIRE(vs[3] == 1 || vs[2] == 1,
                "attn_fwd: v needs unit stride along head_dim or along the sequence");
  HYDRA_REQUIRE(hd <= 256, "attn_fwd: head_dim must be <= 256");
  HYDRA_REQUIRE(mask_mode >= HYDRA_MASK_NONE && mask_mode <= HYDRA_MASK_REFERENCE_SDPA,
                "attn_fwd: unknown mask mode");
  HYDRA_REQUIRE(mask_mode == HYDRA_MASK_NONE || key_mask != nullptr || need,
                "attn_fwd: mask mode needs key_mask");
  HYDRA_REQUIRE(workspace_bytes >= 0, "attn_fwd: negative workspace size");
  HYDRA_REQUIRE(mask_mode != HYDRA_MASK_REFERENCE_SDPA || causal,
                "attn_fwd: the reference-SDPA mask mode is defined with causal=1");
  if (B * S == 0) return HYDRA_OK;
  HYDRA_REQUIRE(need || (q && k && v && o), "attn_fwd: null pointer");
  HYDRA_REQUIRE(S < (int64_t(1) << 30), "attn_fwd: sequence too long");
  const uint8_t* km = mask_mode == HYDRA_MASK_NONE ? nullptr : key_mask;
  auto st = static_cast<hipStream_t>(stream);
  const bool mfma_shape = (hd == 16 || hd == 32 || hd == 64 || hd == 128);
  bool strides8 = true;
  for (int i = 0; i < 3; ++i)
    strides8 = strides8 && qs[i] % 8 == 0 && ks[i] % 8 == 0 && os[i] % 4 == 0;
  // The bf16 kernel addresses a K/V tile with 32-bit byte offsets from a
  // per-tile base, and relies on rows that do not overlap.
  const int64_t lim = int64_t(1) << 30;
  strides8 = strides8 && ks[2] >= hd && ks[2] * 2 * 64 < lim;
  if (vs[3] == 1) {
    strides8 = strides8 && vs[0] % 8 == 0 && vs[1] % 8 == 0 && vs[2] % 8 == 0 && vs[2] >= hd &&
               vs[2] * 2 * 64 < lim;
  } else {  // V^T rows: 16-byte chunks of 8 keys, so S must be a multiple of 8
    strides8 = strides8 && vs[0] % 8 == 0 && vs[1] % 8 == 0 && vs[3] % 8 == 0 && S % 8 == 0 &&
               vs[3] >= S && hd * vs[3] * 2 < lim;
  }
  if (dtype == HYDRA_BF16 && mfma_shape && strides8 &&
      (need || (aligned16(q) && aligned16(k) && aligned16(v) && (reinterpret_cast<uintptr_t>(o) & 7u) == 0))) {
    switch (hd) {
      case 16: return launch_mfma<16>(q, k, v, o, lse, km, mask_mode, B, Hq, Hkv, S, qs, ks, vs, os, causal != 0, scale, score_bound, bound_temperature, bound_temperature_dtype == HYDRA_BF16 ? 1 : 0, workspace, static_cast<size_t>(workspace_bytes), need, st);
      case 32: return launch_mfma<32>(q, k, v, o, lse, km, mask_mode, B, Hq, Hkv, S, qs, ks, vs, os, causal != 0, scale, score_bound, bound_temperature, bound_temperature_dtype == HYDRA_BF16 ? 1 : 0, workspace, static_cast<size_t>(workspace_bytes), need, st);
      case 64: return launch_mfma<64>(q, k, v, o, lse, km, mask_mode, B, Hq, Hkv, S, qs, ks, vs, os, causal != 0, scale, score_bound, bound_temperature, bound_temperature_dtype == HYDRA_BF16 ? 1 : 0, workspace, static_cast<size_t>(workspace_bytes), need, st);
      default: return launch_mfma<128>(q, k, v, o, lse, km, mask_mode, B, Hq, Hkv, S, qs, ks, vs, os, causal != 0, scale, score_bound, bound_temperature, bound_temperature_dtype == HYDRA_BF16 ? 1 : 0, workspace, static_cast<size_t>(workspace_bytes), need, st);
    }
  }
  HYDRA_REQUIRE(B * Hq * S / 256 < (int64_t(1) << 31), "attn_fwd: too many rows");
  if (need) return HYDRA_OK;  // the VALU kernels take no scratch
  const bool split_shape = hd == 8 || hd == 16 || hd == 32 || hd == 64 || hd == 128;
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    if (split_shape && getenv("HYDRA_ATTN_GENERIC") == nullptr)
      return launch_split<T>(q, k, v, o, lse, km, mask_mode, B, Hq, Hkv, S, hd, qs, ks, vs, os,
                             causal != 0, scale, st);
    return launch_generic<T>(q, k, v, o, lse, km, mask_mode, B, Hq, Hkv, S, hd, qs, ks, vs,
                             os, causal != 0, scale, st);
  });
}

extern "C" int hydra_attn_fwd(const void* q, const void* k, const void* v, void* o,
                              float* lse, const uint8_t* key_mask, int mask_mode,
                              int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t hd,
                              const int64_t* qs, const int64_t* ks, const int64_t* vs,
                              const int64_t* os, int causal, float scale,
                              float score_bound, const void* bound_temperature,
                              int bound_temperature_dtype, int dtype, void* workspace,
                              int64_t workspace_bytes, void* stream) {
  return attn_fwd_impl(q, k, v, o, lse, key_mask, mask_mode, B, Hq, Hkv, S, hd, qs, ks, vs, os, causal,
                       scale, score_bound, bound_temperature, bound_temperature_dtype, dtype, workspace,
                       workspace_bytes, nullptr, stream);
}

extern "C" int hydra_attn_fwd_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t hd,
                                        const int64_t* qs, const int64_t* ks, const int64_t* vs,
                                        const int64_t* os, int causal, int mask_mode, int dtype,
                                        int64_t* bytes) {
  HYDRA_REQUIRE(bytes != nullptr, "attn_fwd_workspace: null result pointer");
  size_t need = 0;
  const int rc = attn_fwd_impl(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, mask_mode, B, Hq, Hkv, S,
                               hd, qs, ks, vs, os, causal, 1.f, 0.f, nullptr, HYDRA_F32, dtype, nullptr, 0,
                               &need, nullptr);
  *bytes = static_cast<int64_t>(need);
  return rc;
}
