// CCGQA attention backward on gfx950: the gradients of
// o = softmax(scale * q k^T [+ causal mask]) v with respect to q, k and v,
// K/V heads shared by G = Hq/Hkv query heads in repeat_interleave order.
// Reference semantics: CCGQAAttentionFused.backward
// (hydra/attention/backends/ccgqa/kernels/fused_attention.py:706-823) and its
// split-K kernels _bwd_gqa_kv_kernel / _bwd_gqa_dq_kernel (:113-338) and
// _bwd_kernel / _bwd_dq_kernel (:432-635): P is recomputed from the
// forward's log-sum-exp, D = rowsum(dO * O), dS = P (dP - D) scale with
// dP = dO V^T, dV = sum_g P_g^T dO_g, dK = sum_g dS_g^T Q_g, dQ = dS K.
// fp32 accumulation, one rounding per output, no atomics: every launch is
// deterministic.
//
// Launches on the bf16 path (v_mfma_f32_32x32x16_bf16):
//  * attn_bwd_rowdot_kernel: D and lse * log2(e) per query row (fp32).
//  * attn_bwd_dkdv_kernel: lanes own keys.  A workgroup is KB key blocks of
//    32 keys x HG head groups (one wave each); a step stages 32 query rows
//    of Q and dO for HG heads in LDS, row-major (A operand of S = Q K^T and
//    dP = dO V^T) and transposed (A operand of dV^T += dO^T P and
//    dK^T += Q^T dS), so the KB waves of a head group share each staged
//    tile.  K and V fragments stay in registers for the whole walk; at the
//    end the head groups' partial dK/dV are summed through LDS in a fixed
//    order.  Workgroups start with the lowest keys (the longest causal
//    walks); with few key groups each one's query range is cut into
//    chunks whose fp32 partials attn_bwd_dkdv_reduce_kernel sums in order.
//  * attn_bwd_dq_kernel: lanes own queries, as in the forward: S^T = K Q^T,
//    dP^T = V dO^T, dQ^T += K^T dS^T; a step stages 64 keys of K and V
//    (row-major) and K^T in LDS, shared by the 4 query tasks of an item.
//    It runs on a side stream, concurrently with dK/dV (see SideStream).
// The MFMA B operand of the PV-type products is taken straight from the
// score accumulator registers; the A operand is read from the transposed
// LDS tile in the same (register-order) permutation of the summed index.
// Generic path (attn_bwd_generic_*): one thread per query / key row, fp32
// math, any element type, head_dim <= 256.
#include "common.h"

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <type_traits>

namespace hydra {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kDqWaves = 4;    // query tasks (waves) per dQ workgroup
constexpr int kVmcnt0 = 0x3f70;  // s_waitcnt vmcnt(0), expcnt/lgkmcnt untouched (gfx9 encoding)

__device__ __forceinline__ f32x16_t mfma(uint4 a, uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int r = 0; r < 16; ++r) z[r] = 0.f;
  return z;
}

// Registers base..base+7 of a C tile as a bf16 B fragment.  Register r of a
// 32x32 C tile holds row 8(r/4) + 4hf + r%4, so this fragment's 8 k-values
// are rows 16c + 4hf + 0..3 and 16c + 8 + 4hf + 0..3 (c = base / 8).
__device__ __forceinline__ uint4 pack_c8(const f32x16_t& x, int base) {
  return make_uint4(pack2<bf16>(x[base + 0], x[base + 1]), pack2<bf16>(x[base + 2], x[base + 3]),
                    pack2<bf16>(x[base + 4], x[base + 5]), pack2<bf16>(x[base + 6], x[base + 7]));
}

// A fragment from a transposed LDS tile t[row][col] (pitch in elements),
// with the columns in the permutation pack_c8 gives the k index: lane
// (n, hf) takes row `row`, columns 16c + 4hf + 0..3 and 16c + 8 + 4hf + 0..3.
__device__ __forceinline__ uint4 lds_a_perm(const uint16_t* t, int row, int pitch, int c, int hf) {
  const uint16_t* p = t + row * pitch + 16 * c + 4 * hf;
  const uint2 lo = *reinterpret_cast<const uint2*>(p);
  const uint2 hi = *reinterpret_cast<const uint2*>(p + 8);
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// Element i of two 16-byte rows a and b as one 32-bit word (a_i | b_i << 16).
__device__ __forceinline__ uint32_t pair_word(const uint4& a, const uint4& b, int i) {
  const uint32_t wa = i < 2 ? a.x : i < 4 ? a.y : i < 6 ? a.z : a.w;
  const uint32_t wb = i < 2 ? b.x : i < 4 ? b.y : i < 6 ? b.z : b.w;
  return (i & 1) ? (wa >> 16) | (wb & 0xffff0000u) : (wa & 0xffffu) | (wb << 16);
}

// Writes the 8 d-values of rows 2p and 2p+1 (chunk c) into a transposed tile
// t[d][row] as 8 words.
__device__ __forceinline__ void st_pair_t(uint16_t* t, int pitch, int c, int p, const uint4& a,
                                          const uint4& b) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
    *reinterpret_cast<uint32_t*>(&t[(8 * c + i) * pitch + 2 * p]) = pair_word(a, b, i);
}

// Buffer resource over `bytes` bytes from `base`: loads past the end return
// zero (hardware range check), so tiles that overhang S need no branches --
// which also keeps the compiler's vmcnt bookkeeping exact across the
// prefetch.
constexpr int kRsrcFlags = 0x00020000;  // raw (untyped) access, gfx9 family
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           kRsrcFlags);
}
__device__ __forceinline__ uint4 ld16_buf(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ float ld4_buf(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

__device__ __forceinline__ uint4 ld16_or0(const bf16* p, bool ok) {
  return ok ? *reinterpret_cast<const uint4*>(p) : make_uint4(0, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// D[r] = sum_d dO[r,d] O[r,d] and lse2[r] = lse[r] * log2(e), r = (b*Hq+h)*S+s.
// blockIdx.y + 65535 blockIdx.z = b*Hq+h; TPR threads per row, each a
// strided set of E-element chunks (ONE: the launch made hd <= TPR * E, one
// chunk per thread); a thread group takes RPG consecutive rows, all of
// their loads issued before the sums.
template <typename T, int TPR, bool VEC, int RPG, bool ONE>
__global__ __launch_bounds__(256) void attn_bwd_rowdot_kernel(
    const T* __restrict__ o, const T* __restrict__ dout, const float* __restrict__ lse,
    float* __restrict__ dvec, float* __restrict__ lse2, int BH, int Hq, int S, int hd,
    int64_t os0, int64_t os1, int64_t os2, int64_t ds0, int64_t ds1, int64_t ds2) {
  constexpr int E = VEC ? 16 / int(sizeof(T)) : 1;
  const int bh = blockIdx.y + 65535 * blockIdx.z;
  if (bh >= BH) return;
  const int b = bh / Hq, h = bh - b * Hq;
  const int s0 = ((blockIdx.x * 256 + threadIdx.x) / TPR) * RPG;
  const int sub = threadIdx.x % TPR;
  const T* obase = o + b * os0 + h * os1;
  const T* dbase = dout + b * ds0 + h * ds1;
  float acc[RPG];
  if constexpr (ONE && VEC) {
    // hd <= TPR * E: one 16-byte chunk of each row per thread, all loaded first
    float a[RPG][E], c[RPG][E];
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
      const int s = s0 + j, e = sub * E;
      if (s < S && e < hd) {
        load16<T>(obase + static_cast<int64_t>(s) * os2 + e, a[j]);
        load16<T>(dbase + static_cast<int64_t>(s) * ds2 + e, c[j]);
      } else {
#pragma unroll
        for (int i = 0; i < E; ++i) a[j][i] = c[j][i] = 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
      acc[j] = 0.f;
#pragma unroll
      for (int i = 0; i < E; ++i) acc[j] = fmaf(a[j][i], c[j][i], acc[j]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < RPG; ++j) {
      acc[j] = 0.f;
      const int s = s0 + j;
      if (s >= S) continue;
      const T* orow = obase + static_cast<int64_t>(s) * os2;
      const T* drow = dbase + static_cast<int64_t>(s) * ds2;
      for (int e = sub * E; e < hd; e += TPR * E) {
        if constexpr (VEC) {
          float a[E], c[E];
          load16<T>(orow + e, a);
          load16<T>(drow + e, c);
#pragma unroll
          for (int i = 0; i < E; ++i) acc[j] = fmaf(a[i], c[i], acc[j]);
        } else {
          acc[j] = fmaf(to_f32(orow[e]), to_f32(drow[e]), acc[j]);
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < RPG; ++j) {
    const float v = wave_sum<TPR>(acc[j]);
    const int s = s0 + j;
    if (s < S && sub == 0) {
      const int64_t r = static_cast<int64_t>(bh) * S + s;
      dvec[r] = v;
      lse2[r] = lse[r] * kLog2e;
    }
  }
}

// ---------------------------------------------------------------------------
// dK/dV, lanes own keys (bf16, MFMA).
template <int HD>
struct DkdvLayout {
  static constexpr int QP = HD + 8;          // row-major pitch (elements): 16-byte rows, 4-bank skew
  static constexpr int TP = 32 + 4;          // transposed pitch (elements)
  static constexpr int ROWS = 32 * QP;       // one row-major 32-row tile
  static constexpr int TRS = HD * TP;        // one transposed tile
  static constexpr int HGE = 2 * ROWS + 2 * TRS + 2 * 32 * 2;  // Q, dO, Q^T, dO^T, lse2, D (elements)
};

template <int HD, bool CAUSAL, int KB, int HG>
__global__ __launch_bounds__(64 * KB * HG) void attn_bwd_dkdv_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ dout, const float* __restrict__ dvec, const float* __restrict__ lse2,
    bf16* __restrict__ dk, bf16* __restrict__ dv, float* __restrict__ part, int Hq, int Hkv,
    int S, int G, int nwg, int ch, int maxch,
    int64_t qs0, int64_t qs1, int64_t qs2, int64_t ks0, int64_t ks1, int64_t ks2,
    int64_t vs0, int64_t vs1, int64_t vs2, int64_t ds0, int64_t ds1, int64_t ds2,
    int64_t dks0, int64_t dks1, int64_t dks2, int64_t dvs0, int64_t dvs1, int64_t dvs2,
    float scale_log2, float scale) {
  constexpr int NT = 64 * KB * HG;
  constexpr int KS = HD / 16;   // k-steps over head_dim
  constexpr int DT = HD / 32;   // 32-row d tiles of dK^T / dV^T
  constexpr int DC = HD / 8;    // 16-byte chunks per row
  using L = DkdvLayout<HD>;
  constexpr int STAGE = HG * L::HGE;
  constexpr int UNITS = HG * 16 * DC;         // (head group, row pair, chunk) staging units
  constexpr int UPT = (UNITS + NT - 1) / NT;
  constexpr int FOLD = (HG - 1) * KB * 64 * 2 * DT * 16;  // floats exchanged at the end
  constexpr int SMEM = 2 * STAGE > FOLD * 2 ? 2 * STAGE : FOLD * 2;
  __shared__ __attribute__((aligned(16))) uint16_t smem[SMEM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: per-wave branches stay uniform
  const int n = lane & 31, hf = lane >> 5;
  const int kbl = wave % KB, hg = wave / KB;
  const int BHkv = gridDim.x / nwg;
  const int bk = blockIdx.x % BHkv;
  const int b = bk / Hkv, kvh = bk - b * Hkv;
  const int nkg = (S + 32 * KB - 1) / (32 * KB);
  const int nqt = (S + 31) / 32;
  // Workgroup -> (key group kg, chunk): each key group's nq query tiles
  // are cut into ceil(nq / ch) chunks of ch tiles.  Without chunking
  // (ch >= nqt) the key groups come in order, the longest causal walks
  // first.  With chunking the order is longest first over all chunks, so
  // that the dispatcher's next-free-CU assignment is a longest-processing-
  // time schedule: every full chunk (key groups in order), then the partial
  // chunks by decreasing length.  Their lengths nq mod ch repeat with
  // period T = ch / gcd(ch, KB) in kg (causal; 1 otherwise), so the partial
  // chunks are taken class by class (kg = j, j + T, ...), classes by
  // decreasing remainder.  Scalar loops: nkg, then (ch - 1) x T <= 240
  // iterations (the host chunks with ch <= 16).
  auto nq_of = [&](int g) { return CAUSAL ? nqt - KB * g : nqt; };
  int kg = -1, chunk = static_cast<int>(blockIdx.x) / BHkv;
  if (ch >= nqt) {
    for (kg = 0; kg + 1 < nkg; ++kg) {
      const int c = (nq_of(kg) + ch - 1) / ch;
      if (chunk < c) break;
      chunk -= c;
    }
  } else {
    for (int g = 0; g < nkg; ++g) {
      const int f = nq_of(g) / ch;
      if (chunk < f) {
        kg = g;
        break;
      }
      chunk -= f;
    }
    if (kg < 0) {
      int a = ch, c = KB;  // gcd(ch, KB)
      while (c) {
        const int t = a % c;
        a = c;
        c = t;
      }
      const int T = CAUSAL ? ch / a : 1;
      for (int r = ch - 1; r >= 1 && kg < 0; --r)
        for (int j = 0; j < T && j < nkg && kg < 0; ++j) {
          if (nq_of(j) % ch != r) continue;
          const int cnt = (nkg - j + T - 1) / T;
          if (chunk < cnt) kg = j + chunk * T;
          else chunk -= cnt;
        }
      kg = max(kg, 0);  // not reached: the host launches exactly the chunk count
      chunk = nq_of(kg) / ch;
    }
  }
  const int nch = (nq_of(kg) + ch - 1) / ch;
  const int kg0 = 32 * KB * kg;           // first key of the workgroup
  const int kw0 = kg0 + 32 * kbl;         // first key of this wave
  const int key = kw0 + n;

  // K and V fragments (B operands of S = Q K^T, dP = dO V^T).
  uint4 kf[KS], vf[KS];
  {
    const bool ok = key < S;
    const bf16* kr = k + b * ks0 + kvh * ks1 + static_cast<int64_t>(ok ? key : 0) * ks2;
    const bf16* vr = v + b * vs0 + kvh * vs1 + static_cast<int64_t>(ok ? key : 0) * vs2;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      kf[s] = ld16_or0(kr + 16 * s + 8 * hf, ok);
      vf[s] = ld16_or0(vr + 16 * s + 8 * hf, ok);
    }
  }
  // Retire these loads before the loop: the in-order vmcnt would otherwise
  // make the loop's first use of kf/vf wait for the tile prefetches too.
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
  f32x16_t dka[DT], dva[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) { dka[dt] = zero16(); dva[dt] = zero16(); }

  const int qt0 = (CAUSAL ? KB * kg : 0) + chunk * ch;  // this chunk's query tiles
  const int nq = min(ch, nqt - qt0);
  const int rounds = G / HG;
  const int nsteps = rounds * nq;
  // Step order: round-major over the chunk's query tiles, except that when
  // the chunk starts with all KB tiles that hold the waves' diagonals
  // (tiles KB kg .. KB kg + KB - 1), those come first for every round
  // (steps [0, ediag)), so the remaining steps run the unmasked tile code
  // only.  A chunk holding only part of that region (chunks shorter than
  // KB tiles) takes the masking dispatch for every step.
  const int dreg = CAUSAL ? max(0, min(KB * kg + KB - qt0, nq)) : 0;
  const int nd = dreg == KB ? KB : 0;
  const int nr = max(nq - nd, 1);
  const int ediag = nd ? rounds * nd : (dreg > 0 ? nsteps : 0);
  auto locate = [&](int step, int& hr, int& qt) {
    if (step < rounds * nd) {
      hr = step / nd;
      qt = qt0 + (step - hr * nd);
    } else {
      const int s2 = step - rounds * nd;
      hr = s2 / nr;
      qt = qt0 + nd + (s2 - hr * nr);
    }
  };

  // Staging registers: per unit the chunk c of rows 2p, 2p+1 of Q and dO.
  struct Regs {
    uint4 q[UPT][2], d[UPT][2];
    float l, dv;  // lse2 / D of one row (threads < 32 * HG)
  };
  Regs ra, rb;
  auto fetch = [&](int step, Regs& R) {
    int hr, qt;
    locate(step, hr, qt);
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const int unit = tid + NT * u;
      if (UNITS % NT == 0 || unit < UNITS) {
        // 16 * DC >= 64 units share a head group, so g is wave-uniform (and
        // the buffer resources below scalar).
        const int g = __builtin_amdgcn_readfirstlane(unit / (16 * DC));
        const int rem = unit - g * (16 * DC);
        const int c = rem >> 4, p = rem & 15;  // p fastest: conflict-free transposed writes
        const int h = kvh * G + hr * HG + g;
        const int r0 = 32 * qt + 2 * p;  // rows >= S read as zero
        const auto qr = rows_rsrc(q + b * qs0 + h * qs1, (S - 1) * qs2 * 2 + HD * 2);
        const auto dr = rows_rsrc(dout + b * ds0 + h * ds1, (S - 1) * ds2 * 2 + HD * 2);
        const int qo = r0 * static_cast<int>(qs2) * 2 + 16 * c;
        const int dof = r0 * static_cast<int>(ds2) * 2 + 16 * c;
        R.q[u][0] = ld16_buf(qr, qo);
        R.q[u][1] = ld16_buf(qr, qo + static_cast<int>(qs2) * 2);
        R.d[u][0] = ld16_buf(dr, dof);
        R.d[u][1] = ld16_buf(dr, dof + static_cast<int>(ds2) * 2);
      }
    }
    {
      // Rows of this round's HG heads (threads < 32 HG); rows past S, and
      // the other threads, read lse2 = D = 0 through an out-of-range offset
      // (with zero Q and dO rows such rows add nothing: dS = P (0 - 0) = 0
      // and dO^T P = 0).  Every thread issues the same loads, so the
      // compiler's vmcnt bookkeeping stays exact.
      const int g = tid >> 5, row = 32 * qt + (tid & 31);
      const int64_t h0 = static_cast<int64_t>(b) * Hq + kvh * G + hr * HG;
      const int off = (tid < 32 * HG && row < S) ? (g * S + row) * 4 : 0x7ffffff0;
      R.l = ld4_buf(rows_rsrc(lse2 + h0 * S, int64_t(HG) * S * 4), off);
      R.dv = ld4_buf(rows_rsrc(dvec + h0 * S, int64_t(HG) * S * 4), off);
    }
  };
  auto land = [&](int buf, const Regs& R) {
    uint16_t* st = smem + buf * STAGE;
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const int unit = tid + NT * u;
      if (UNITS % NT == 0 || unit < UNITS) {
        const int g = unit / (16 * DC), rem = unit - g * (16 * DC);
        const int c = rem >> 4, p = rem & 15;  // p fastest: conflict-free transposed writes
        uint16_t* hb = st + g * L::HGE;
        *reinterpret_cast<uint4*>(&hb[(2 * p) * L::QP + 8 * c]) = R.q[u][0];
        *reinterpret_cast<uint4*>(&hb[(2 * p + 1) * L::QP + 8 * c]) = R.q[u][1];
        *reinterpret_cast<uint4*>(&hb[L::ROWS + (2 * p) * L::QP + 8 * c]) = R.d[u][0];
        *reinterpret_cast<uint4*>(&hb[L::ROWS + (2 * p + 1) * L::QP + 8 * c]) = R.d[u][1];
        st_pair_t(hb + 2 * L::ROWS, L::TP, c, p, R.q[u][0], R.q[u][1]);
        st_pair_t(hb + 2 * L::ROWS + L::TRS, L::TP, c, p, R.d[u][0], R.d[u][1]);
      }
    }
    if (tid < 32 * HG) {
      float* f = reinterpret_cast<float*>(st + (tid >> 5) * L::HGE + 2 * L::ROWS + 2 * L::TRS);
      f[tid & 31] = R.l;
      f[32 + (tid & 31)] = R.dv;
    }
  };

  // One 32-query tile; DIAG: the tile on this wave's diagonal (key <= query mask).
  auto tile = [&](auto diag_tag, int q0, int buf) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    {
      const uint16_t* hb = smem + buf * STAGE + hg * L::HGE;
      const uint16_t* Qs = hb;
      const uint16_t* Ds = hb + L::ROWS;
      const uint16_t* Qt = hb + 2 * L::ROWS;
      const uint16_t* Dt = Qt + L::TRS;
      const float* lsv = reinterpret_cast<const float*>(Dt + L::TRS);
      f32x16_t s = zero16(), dp = zero16();
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint4 aq = *reinterpret_cast<const uint4*>(&Qs[n * L::QP + 16 * ks + 8 * hf]);
        s = mfma(aq, kf[ks], s);
        const uint4 ad = *reinterpret_cast<const uint4*>(&Ds[n * L::QP + 16 * ks + 8 * hf]);
        dp = mfma(ad, vf[ks], dp);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 l4 = *reinterpret_cast<const float4*>(&lsv[8 * j + 4 * hf]);
        const float4 d4 = *reinterpret_cast<const float4*>(&lsv[32 + 8 * j + 4 * hf]);
        const float lj[4] = {l4.x, l4.y, l4.z, l4.w};
        const float dj[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * j + i;
          float p = __builtin_amdgcn_exp2f(fmaf(s[r], scale_log2, -lj[i]));
          if constexpr (DIAG) p = (key <= q0 + 8 * j + 4 * hf + i) ? p : 0.f;
          s[r] = p;
          dp[r] = p * (dp[r] - dj[i]);
        }
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const uint4 pb = pack_c8(s, 8 * c);
        const uint4 sb = pack_c8(dp, 8 * c);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          dva[dt] = mfma(lds_a_perm(Dt, 32 * dt + n, L::TP, c, hf), pb, dva[dt]);
          dka[dt] = mfma(lds_a_perm(Qt, 32 * dt + n, L::TP, c, hf), sb, dka[dt]);
        }
      }
    }
  };
  auto compute = [&](int step, int buf) {
    int hr, qt;
    locate(step, hr, qt);
    const int q0 = 32 * qt;
    // Causal: the tile reaches this wave's keys iff q0 + 31 >= kw0; only
    // the diagonal tile q0 == kw0 needs the key <= query mask.
    if (CAUSAL && q0 == kw0) tile(std::true_type{}, q0, buf);
    else if (!CAUSAL || q0 > kw0) tile(std::false_type{}, q0, buf);
  };

  // Two register sets alternate, so a tile's loads have two steps to land.
  // Fetches are unconditional (past the end they repeat the last tile) so
  // that every path issues the same loads and each land() waits only for
  // its own set.
  const int last = nsteps - 1;  // >= 0
  fetch(0, ra);
  land(0, ra);
  fetch(min(1, last), rb);
  __syncthreads();
  // Past ediag every wave is strictly below the diagonal: tile<false> only,
  // in a loop of its own (no masked path to join, so no accumulator copies).
  auto unmasked = [&](int step, int buf) {
    int hr, qt;
    locate(step, hr, qt);
    tile(std::false_type{}, 32 * qt, buf);
  };
  int step = 0;
  for (; step < last && step + 1 < ediag; step += 2) {  // ediag is even or nsteps
    fetch(min(step + 2, last), ra);
    compute(step, 0);
    land(1, rb);
    __syncthreads();
    fetch(min(step + 3, last), rb);
    compute(step + 1, 1);
    land(0, ra);
    __syncthreads();
  }
  for (; step < last; step += 2) {
    fetch(min(step + 2, last), ra);
    unmasked(step, 0);
    land(1, rb);
    __syncthreads();
    fetch(min(step + 3, last), rb);
    unmasked(step + 1, 1);
    land(0, ra);
    __syncthreads();
  }
  if (step == last) compute(step, 0);  // odd count: the last tile is in buffer 0
  __syncthreads();  // the fold below reuses the staging buffers

  // Fold the head groups (fixed order: group 0 + group 1 + ...), then store.
  float* xf = reinterpret_cast<float*>(smem);
  if constexpr (HG > 1) {
    if (hg > 0) {
      float* dst = xf + (((hg - 1) * KB + kbl) * 2 * DT * 16) * 64;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          dst[((2 * dt) * 16 + r) * 64 + lane] = dka[dt][r];
          dst[((2 * dt + 1) * 16 + r) * 64 + lane] = dva[dt][r];
        }
    }
    __syncthreads();
    if (hg == 0) {
#pragma unroll
      for (int g = 1; g < HG; ++g) {
        const float* src = xf + (((g - 1) * KB + kbl) * 2 * DT * 16) * 64;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            dka[dt][r] += src[((2 * dt) * 16 + r) * 64 + lane];
            dva[dt][r] += src[((2 * dt + 1) * 16 + r) * 64 + lane];
          }
      }
    }
  }
  if (nch > 1) {
    // One of several chunks: fp32 partials, summed in chunk order by
    // attn_bwd_dkdv_reduce_kernel.
    if (hg == 0 && key < S) {
      float* pk = part + ((static_cast<int64_t>(bk) * nkg + kg) * maxch + chunk) * (KB * 32 * HD * 2) +
                  (32 * kbl + n) * HD;
      float* pv = pk + KB * 32 * HD;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d = 32 * dt + 8 * j + 4 * hf;
          *reinterpret_cast<float4*>(pk + d) =
              make_float4(dka[dt][4 * j], dka[dt][4 * j + 1], dka[dt][4 * j + 2], dka[dt][4 * j + 3]);
          *reinterpret_cast<float4*>(pv + d) =
              make_float4(dva[dt][4 * j], dva[dt][4 * j + 1], dva[dt][4 * j + 2], dva[dt][4 * j + 3]);
        }
    }
  } else if (hg == 0 && key < S) {
    bf16* kr = dk + b * dks0 + kvh * dks1 + static_cast<int64_t>(key) * dks2;
    bf16* vr = dv + b * dvs0 + kvh * dvs1 + static_cast<int64_t>(key) * dvs2;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * dt + 8 * j + 4 * hf;
        const f32x16_t& a = dka[dt];
        const f32x16_t& c = dva[dt];
        *reinterpret_cast<uint2*>(kr + d) =
            make_uint2(pack2<bf16>(a[4 * j] * scale, a[4 * j + 1] * scale),
                       pack2<bf16>(a[4 * j + 2] * scale, a[4 * j + 3] * scale));
        *reinterpret_cast<uint2*>(vr + d) =
            make_uint2(pack2<bf16>(c[4 * j], c[4 * j + 1]), pack2<bf16>(c[4 * j + 2], c[4 * j + 3]));
      }
  }
}

// Sums the chunk partials of key groups that were split (in chunk order),
// scales dK and writes both gradients; one thread per 4 values of a key
// row, blockIdx.y + 65535 blockIdx.z = b * Hkv + kv head.  The loads of 8
// chunks are issued before they are added (in order), so a thread waits
// for one load latency per 8 chunks.
template <int HD, bool CAUSAL, int KB>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_reduce_kernel(
    const float* __restrict__ part, bf16* __restrict__ dk, bf16* __restrict__ dv, int BHkv, int Hkv,
    int S, int ch, int maxch, int64_t dks0, int64_t dks1, int64_t dks2, int64_t dvs0, int64_t dvs1,
    int64_t dvs2, float scale) {
  constexpr int CS = KB * 32 * HD * 2;  // floats per chunk partial (dK, then dV)
  constexpr int U = 8;
  const int bk = blockIdx.y + 65535 * blockIdx.z;
  const int i = blockIdx.x * 256 + threadIdx.x;  // < S * HD / 4
  if (bk >= BHkv || i >= S * (HD / 4)) return;
  const int d = 4 * (i % (HD / 4));
  const int key = i / (HD / 4);
  const int nkg = (S + 32 * KB - 1) / (32 * KB), nqt = (S + 31) / 32;
  const int kg = key / (32 * KB);
  const int nch = ((CAUSAL ? nqt - KB * kg : nqt) + ch - 1) / ch;
  if (nch <= 1) return;
  const float* pk = part + (static_cast<int64_t>(bk) * nkg + kg) * maxch * CS + (key - 32 * KB * kg) * HD + d;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f), c = a;
  for (int j0 = 0; j0 < nch; j0 += U) {
    float4 x[U], y[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (j0 + u < nch) {
        x[u] = *reinterpret_cast<const float4*>(pk + static_cast<int64_t>(j0 + u) * CS);
        y[u] = *reinterpret_cast<const float4*>(pk + static_cast<int64_t>(j0 + u) * CS + KB * 32 * HD);
      }
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (j0 + u < nch) {
        a.x += x[u].x; a.y += x[u].y; a.z += x[u].z; a.w += x[u].w;
        c.x += y[u].x; c.y += y[u].y; c.z += y[u].z; c.w += y[u].w;
      }
  }
  const int b = bk / Hkv, kvh = bk - b * Hkv;
  *reinterpret_cast<uint2*>(dk + b * dks0 + kvh * dks1 + key * dks2 + d) =
      make_uint2(pack2<bf16>(a.x * scale, a.y * scale), pack2<bf16>(a.z * scale, a.w * scale));
  *reinterpret_cast<uint2*>(dv + b * dvs0 + kvh * dvs1 + key * dvs2 + d) =
      make_uint2(pack2<bf16>(c.x, c.y), pack2<bf16>(c.z, c.w));
}

// ---------------------------------------------------------------------------
// dQ, lanes own queries (bf16, MFMA).
template <int HD>
struct DqLayout {
  static constexpr int BN = 64;              // keys per step
  static constexpr int KP = HD + 8;          // row-major pitch (elements)
  static constexpr int TP = BN + 4;          // transposed pitch (elements)
  static constexpr int ROWS = BN * KP;
  static constexpr int TRS = HD * TP;
  static constexpr int STAGE = 2 * ROWS + TRS;  // K, V, K^T
};

template <int HD, bool CAUSAL, int NW>
__global__ __launch_bounds__(64 * NW) void attn_bwd_dq_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const bf16* __restrict__ dout, const float* __restrict__ dvec, const float* __restrict__ lse2,
    bf16* __restrict__ dq, int Hq, int Hkv, int S, int G, int ntasks, int items,
    int64_t qs0, int64_t qs1, int64_t qs2, int64_t ks0, int64_t ks1, int64_t ks2,
    int64_t vs0, int64_t vs1, int64_t vs2, int64_t ds0, int64_t ds1, int64_t ds2,
    int64_t dqs0, int64_t dqs1, int64_t dqs2, float scale_log2, float scale) {
  using L = DqLayout<HD>;
  constexpr int BN = L::BN;
  constexpr int MT = BN / 32;
  constexpr int KS = HD / 16;
  constexpr int DT = HD / 32;
  constexpr int DC = HD / 8;
  constexpr int UNITS = (BN / 2) * DC;        // (key pair, chunk) staging units
  constexpr int NT = 64 * NW;
  constexpr int UPT = (UNITS + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * L::STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: per-wave branches stay uniform
  const int n = lane & 31, hf = lane >> 5;
  const int BHkv = gridDim.x / items;
  const int bk = blockIdx.x % BHkv;
  const int item = items - 1 - static_cast<int>(blockIdx.x / BHkv);  // longest first
  const int b = bk / Hkv, kvh = bk - b * Hkv;
  const int task = NW * item + wave;
  const bool active = task < ntasks;
  const int qb = (active ? task : ntasks - 1) / G;
  const int h = kvh * G + (active ? task : ntasks - 1) % G;
  const int q0 = 32 * qb, qi = q0 + n;
  const bool qok = active && qi < S;

  // Q (B operand of S^T = K Q^T) and dO (B operand of dP^T = V dO^T) rows.
  uint4 qf[KS], of[KS];
  float l2 = 0.f, dd = 0.f;
  {
    const bf16* qr = q + b * qs0 + h * qs1 + static_cast<int64_t>(qok ? qi : 0) * qs2;
    const bf16* orow = dout + b * ds0 + h * ds1 + static_cast<int64_t>(qok ? qi : 0) * ds2;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qf[s] = ld16_or0(qr + 16 * s + 8 * hf, qok);
      of[s] = ld16_or0(orow + 16 * s + 8 * hf, qok);
    }
    if (qok) {
      const int64_t ri = (static_cast<int64_t>(b) * Hq + h) * S + qi;
      l2 = lse2[ri];
      dd = dvec[ri];
    }
  }
  // Retire these loads before the loop (see attn_bwd_dkdv_kernel).
  __builtin_amdgcn_s_waitcnt(kVmcnt0);
  f32x16_t acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = zero16();

  // Keys the item needs: up to its last query (causal) or all of them.
  const int last_task = min(NW * item + NW - 1, ntasks - 1);
  const int qmax = min(32 * (last_task / G) + 31, S - 1);
  const int nkt = CAUSAL ? qmax / BN + 1 : (S + BN - 1) / BN;
  const int my_last = CAUSAL ? min(q0 + 31, S - 1) : S - 1;  // this wave's last visible key

  const auto krs = rows_rsrc(k + b * ks0 + kvh * ks1, (S - 1) * ks2 * 2 + HD * 2);
  const auto vrs = rows_rsrc(v + b * vs0 + kvh * vs1, (S - 1) * vs2 * 2 + HD * 2);
  struct Regs {
    uint4 k[UPT][2], v[UPT][2];
  };
  Regs ra, rb;
  auto fetch = [&](int kt, Regs& R) {
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const int unit = tid + NT * u;
      if (UNITS % NT == 0 || unit < UNITS) {
        const int c = unit >> 5, p = unit & 31;  // p fastest: conflict-free transposed writes
        const int k0 = BN * kt + 2 * p;  // keys >= S read as zero
        const int ko = k0 * static_cast<int>(ks2) * 2 + 16 * c;
        const int vo = k0 * static_cast<int>(vs2) * 2 + 16 * c;
        R.k[u][0] = ld16_buf(krs, ko);
        R.k[u][1] = ld16_buf(krs, ko + static_cast<int>(ks2) * 2);
        R.v[u][0] = ld16_buf(vrs, vo);
        R.v[u][1] = ld16_buf(vrs, vo + static_cast<int>(vs2) * 2);
      }
    }
  };
  auto land = [&](int buf, const Regs& R) {
    uint16_t* st = smem + buf * L::STAGE;
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const int unit = tid + NT * u;
      if (UNITS % NT == 0 || unit < UNITS) {
        const int c = unit >> 5, p = unit & 31;  // p fastest: conflict-free transposed writes
        *reinterpret_cast<uint4*>(&st[(2 * p) * L::KP + 8 * c]) = R.k[u][0];
        *reinterpret_cast<uint4*>(&st[(2 * p + 1) * L::KP + 8 * c]) = R.k[u][1];
        *reinterpret_cast<uint4*>(&st[L::ROWS + (2 * p) * L::KP + 8 * c]) = R.v[u][0];
        *reinterpret_cast<uint4*>(&st[L::ROWS + (2 * p + 1) * L::KP + 8 * c]) = R.v[u][1];
        st_pair_t(st + 2 * L::ROWS, L::TP, c, p, R.k[u][0], R.k[u][1]);
      }
    }
  };

  // One 64-key tile; MASKED: keys past S or after a query of this wave.
  auto tile = [&](auto mask_tag, int key0, int buf) {
    constexpr bool MASKED = decltype(mask_tag)::value;
    {
      const uint16_t* Ks = smem + buf * L::STAGE;
      const uint16_t* Vs = Ks + L::ROWS;
      const uint16_t* Kt = Ks + 2 * L::ROWS;
      f32x16_t st[MT], dp[MT];
      // MASKED: key = key0 + 4 hf + off, off = 32 mt + 8 (r / 4) + r % 4 a
      // constant per register, visible iff off <= lim
      const int lim = (CAUSAL ? min(qi, S - 1) : S - 1) - key0 - 4 * hf;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) { st[mt] = zero16(); dp[mt] = zero16(); }
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int row = (32 * mt + n) * L::KP + 16 * s + 8 * hf;
          st[mt] = mfma(*reinterpret_cast<const uint4*>(&Ks[row]), qf[s], st[mt]);
          dp[mt] = mfma(*reinterpret_cast<const uint4*>(&Vs[row]), of[s], dp[mt]);
        }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float p = __builtin_amdgcn_exp2f(fmaf(st[mt][r], scale_log2, -l2));
          if constexpr (MASKED)  // keys past S, and after the query when causal: P = 0
            p = 32 * mt + 8 * (r >> 2) + (r & 3) <= lim ? p : 0.f;
          dp[mt][r] = p * (dp[mt][r] - dd);
        }
#pragma unroll
      for (int c = 0; c < 2 * MT; ++c) {
        const uint4 sb = pack_c8(dp[c >> 1], 8 * (c & 1));
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          acc[dt] = mfma(lds_a_perm(Kt, 32 * dt + n, L::TP, c, hf), sb, acc[dt]);
      }
    }
  };
  auto compute = [&](int kt, int buf) {
    const int key0 = BN * kt;
    if (!active || key0 > my_last) return;
    if (key0 + BN > S || (CAUSAL && key0 + BN - 1 > q0)) tile(std::true_type{}, key0, buf);
    else tile(std::false_type{}, key0, buf);
  };

  // Two register sets alternate (see attn_bwd_dkdv_kernel).
  const int last = nkt - 1;  // >= 0
  fetch(0, ra);
  land(0, ra);
  fetch(min(1, last), rb);
  __syncthreads();
  // Tiles [0, kt_u) lie below the diagonal of the item's first task and
  // before S, so every active wave takes the unmasked code there, in a loop
  // of its own (kt_u even keeps the two-step pipeline aligned).
  const int q0_first = 32 * ((NW * item) / G);
  const int kt_u = (CAUSAL ? min((q0_first + 1) / BN, S / BN) : S / BN) & ~1;
  int kt = 0;
  for (; kt < last && kt + 1 < kt_u; kt += 2) {
    fetch(min(kt + 2, last), ra);
    if (active) tile(std::false_type{}, BN * kt, 0);
    land(1, rb);
    __syncthreads();
    fetch(min(kt + 3, last), rb);
    if (active) tile(std::false_type{}, BN * (kt + 1), 1);
    land(0, ra);
    __syncthreads();
  }
  for (; kt < last; kt += 2) {
    fetch(min(kt + 2, last), ra);
    compute(kt, 0);
    land(1, rb);
    __syncthreads();
    fetch(min(kt + 3, last), rb);
    compute(kt + 1, 1);
    land(0, ra);
    __syncthreads();
  }
  if (kt == last) compute(kt, 0);  // odd count: the last tile is in buffer 0

  if (qok) {
    bf16* orow = dq + b * dqs0 + h * dqs1 + static_cast<int64_t>(qi) * dqs2;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * dt + 8 * j + 4 * hf;
        const f32x16_t& a = acc[dt];
        *reinterpret_cast<uint2*>(orow + d) =
            make_uint2(pack2<bf16>(a[4 * j] * scale, a[4 * j + 1] * scale),
                       pack2<bf16>(a[4 * j + 2] * scale, a[4 * j + 3] * scale));
      }
  }
}

// ---------------------------------------------------------------------------
// Generic path: fp32 math, one thread per query row (dQ) or key row (dK, dV).
// Rows of up to MAXD elements are accumulated in registers.
// Whether query s sees key t (t < S): causality, then the key mask
// (MASK 1: key padding on top of causality; MASK 2: the forward's
// reference-SDPA mode, key t > s or t padded, whatever `CAUSAL`).
template <bool CAUSAL, int MASK>
__device__ __forceinline__ bool bwd_visible(int s, int t, const uint8_t* kmrow) {
  if constexpr (MASK == 2) return t > s || kmrow[t] == 0;
  const bool c = !CAUSAL || t <= s;
  if constexpr (MASK == 1) return c && kmrow[t] != 0;
  return c;
}

template <typename T, int MAXD, bool CAUSAL, int MASK>
__global__ __launch_bounds__(128) void attn_bwd_generic_dq_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ dout, const float* __restrict__ dvec, const float* __restrict__ lse2,
    const uint8_t* __restrict__ kmask,
    T* __restrict__ dq, int64_t rows, int Hq, int Hkv, int S, int hd,
    int64_t qs0, int64_t qs1, int64_t qs2, int64_t ks0, int64_t ks1, int64_t ks2,
    int64_t vs0, int64_t vs1, int64_t vs2, int64_t ds0, int64_t ds1, int64_t ds2,
    int64_t dqs0, int64_t dqs1, int64_t dqs2, float scale_log2, float scale) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 128 + threadIdx.x;
  if (r >= rows) return;
  const int s = static_cast<int>(r % S);
  const int64_t bh = r / S;
  const int h = static_cast<int>(bh % Hq);
  const int64_t b = bh / Hq;
  const int kvh = h / (Hq / Hkv);
  const T* qr = q + b * qs0 + h * qs1 + s * qs2;
  const T* dr = dout + b * ds0 + h * ds1 + s * ds2;
  constexpr int UNR = MAXD <= 64 ? MAXD : 1;  // longer rows live in scratch anyway
  float qv[MAXD], ov[MAXD], acc[MAXD];
#pragma unroll UNR
  for (int e = 0; e < MAXD; ++e) {
    qv[e] = e < hd ? to_f32(qr[e]) : 0.f;
    ov[e] = e < hd ? to_f32(dr[e]) : 0.f;
    acc[e] = 0.f;
  }
  const float l2 = lse2[r], dd = dvec[r];
  const uint8_t* kmrow = MASK != 0 ? kmask + b * S : nullptr;
  const int tend = CAUSAL && MASK != 2 ? s + 1 : S;
  for (int t = 0; t < tend; ++t) {
    if (MASK != 0 && !bwd_visible<CAUSAL, MASK>(s, t, kmrow)) continue;
    const T* kr = k + b * ks0 + kvh * ks1 + t * ks2;
    const T* vr = v + b * vs0 + kvh * vs1 + t * vs2;
    float sc = 0.f, dpv = 0.f;
#pragma unroll UNR
    for (int e = 0; e < MAXD; ++e)
      if (e < hd) {
        sc = fmaf(qv[e], to_f32(kr[e]), sc);
        dpv = fmaf(ov[e], to_f32(vr[e]), dpv);
      }
    const float p = exp2f(fmaf(sc, scale_log2, -l2));
    const float ds = p * (dpv - dd);
#pragma unroll UNR
    for (int e = 0; e < MAXD; ++e)
      if (e < hd) acc[e] = fmaf(ds, to_f32(kr[e]), acc[e]);
  }
  T* orow = dq + b * dqs0 + h * dqs1 + s * dqs2;
#pragma unroll UNR
  for (int e = 0; e < MAXD; ++e)
    if (e < hd) orow[e] = from_f32<T>(acc[e] * scale);
}

template <typename T, int MAXD, bool CAUSAL, int MASK>
__global__ __launch_bounds__(128) void attn_bwd_generic_dkdv_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ dout, const float* __restrict__ dvec, const float* __restrict__ lse2,
    const uint8_t* __restrict__ kmask,
    T* __restrict__ dk, T* __restrict__ dv, int64_t rows, int Hq, int Hkv, int S, int hd,
    int64_t qs0, int64_t qs1, int64_t qs2, int64_t ks0, int64_t ks1, int64_t ks2,
    int64_t vs0, int64_t vs1, int64_t vs2, int64_t ds0, int64_t ds1, int64_t ds2,
    int64_t dks0, int64_t dks1, int64_t dks2, int64_t dvs0, int64_t dvs1, int64_t dvs2,
    float scale_log2, float scale) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 128 + threadIdx.x;
  if (r >= rows) return;
  const int t = static_cast<int>(r % S);
  const int64_t bk = r / S;
  const int kvh = static_cast<int>(bk % Hkv);
  const int64_t b = bk / Hkv;
  const int G = Hq / Hkv;
  const T* kr = k + b * ks0 + kvh * ks1 + t * ks2;
  const T* vr = v + b * vs0 + kvh * vs1 + t * vs2;
  constexpr int UNR = MAXD <= 64 ? MAXD : 1;  // longer rows live in scratch anyway
  float kv[MAXD], vv[MAXD], ak[MAXD], av[MAXD];
#pragma unroll UNR
  for (int e = 0; e < MAXD; ++e) {
    kv[e] = e < hd ? to_f32(kr[e]) : 0.f;
    vv[e] = e < hd ? to_f32(vr[e]) : 0.f;
    ak[e] = 0.f;
    av[e] = 0.f;
  }
  const uint8_t* kmrow = MASK != 0 ? kmask + b * S : nullptr;
  for (int g = 0; g < G; ++g) {
    const int h = kvh * G + g;
    const int64_t rb = (b * Hq + h) * S;
    for (int s = CAUSAL && MASK != 2 ? t : 0; s < S; ++s) {
      if (MASK != 0 && !bwd_visible<CAUSAL, MASK>(s, t, kmrow)) continue;
      const T* qr = q + b * qs0 + h * qs1 + s * qs2;
      const T* dr = dout + b * ds0 + h * ds1 + s * ds2;
      float sc = 0.f, dpv = 0.f;
#pragma unroll UNR
      for (int e = 0; e < MAXD; ++e)
        if (e < hd) {
          sc = fmaf(to_f32(qr[e]), kv[e], sc);
          dpv = fmaf(to_f32(dr[e]), vv[e], dpv);
        }
      const float p = exp2f(fmaf(sc, scale_log2, -lse2[rb + s]));
      const float ds = p * (dpv - dvec[rb + s]);
#pragma unroll UNR
      for (int e = 0; e < MAXD; ++e)
        if (e < hd) {
          av[e] = fmaf(p, to_f32(dr[e]), av[e]);
          ak[e] = fmaf(ds, to_f32(qr[e]), ak[e]);
        }
    }
  }
  T* okr = dk + b * dks0 + kvh * dks1 + t * dks2;
  T* ovr = dv + b * dvs0 + kvh * dvs1 + t * dvs2;
#pragma unroll UNR
  for (int e = 0; e < MAXD; ++e)
    if (e < hd) {
      okr[e] = from_f32<T>(ak[e] * scale);
      ovr[e] = from_f32<T>(av[e]);
    }
}

struct BwdArgs {
  const void *q, *k, *v, *o, *dout;
  const float* lse;
  void *dq, *dk, *dv;
  int B, Hq, Hkv, S, hd;
  const int64_t *qs, *ks, *vs, *os, *dos, *dqs, *dks, *dvs;
  bool causal;
  float scale;
  hipStream_t st;
  const uint8_t* kmask;  // [B, S], nonzero = keep (mask_mode != 0)
  int mask_mode;
};

template <typename T>
int launch_rowdot(const BwdArgs& a, float* dvec, float* lse2) {
  constexpr int E = 16 / int(sizeof(T));
  const bool vec = a.hd % E == 0 && aligned16(a.o) && aligned16(a.dout) && a.os[0] % E == 0 &&
                   a.os[1] % E == 0 && a.os[2] % E == 0 && a.dos[0] % E == 0 &&
                   a.dos[1] % E == 0 && a.dos[2] % E == 0;
  const T* o = static_cast<const T*>(a.o);
  const T* d = static_cast<const T*>(a.dout);
  constexpr int RPG = 2;
  // rows per block: 256 / TPR thread groups x RPG rows
  const int BH = a.B * a.Hq;
  auto grid = [&](int tpr) {
    return dim3(static_cast<unsigned>((a.S + 256 / tpr * RPG - 1) / (256 / tpr * RPG)),
                static_cast<unsigned>(std::min(BH, 65535)), static_cast<unsigned>((BH + 65534) / 65535));
  };
#define HYDRA_ROWDOT(TPRV, VECV, ONEV)                                                              \
  attn_bwd_rowdot_kernel<T, TPRV, VECV, RPG, ONEV><<<grid(TPRV), 256, 0, a.st>>>(                   \
      o, d, a.lse, dvec, lse2, BH, a.Hq, a.S, a.hd, a.os[0], a.os[1], a.os[2], a.dos[0], a.dos[1],  \
      a.dos[2])
  // vector path: one 16-byte chunk per thread and row when hd <= 16 E
  if (vec && a.hd <= 4 * E) HYDRA_ROWDOT(4, true, true);
  else if (vec && a.hd <= 8 * E) HYDRA_ROWDOT(8, true, true);
  else if (vec && a.hd <= 16 * E) HYDRA_ROWDOT(16, true, true);
  else if (vec) HYDRA_ROWDOT(16, true, false);
  else HYDRA_ROWDOT(16, false, false);
#undef HYDRA_ROWDOT
  return check_launch("attn_bwd: rowdot");
}

// Shape of the dK/dV launch.  Workgroup: KB = 4 blocks of 32 keys x HG
// head groups (G % HG == 0): two head groups (8 waves) when G is even and
// head_dim <= 64, else one.  Four waves share each staged query tile (measured at config 3: 4 x 2
// beats 2 x 4 by 10%, the LDS writes of the staging halve).  With fewer
// than two key groups per CU the query range of each key group is cut into
// chunks of ch tiles (fp32 partials + a reduce launch), so the long causal
// walks of the first key groups spread over more CUs.
struct DkdvPlan {
  int KB, HG, ch, nwg, maxch;
  size_t part_bytes;
};

DkdvPlan plan_dkdv(int hd, int S, int G, int BHkv, bool causal) {
  DkdvPlan p{};
  // two head groups at head_dim 128 spill 631 registers to scratch; one
  // runs that backward 1.75-2.2x faster
  p.HG = G % 2 == 0 && hd <= 64 ? 2 : 1;
  p.KB = 4;
  const int nkg = (S + 32 * p.KB - 1) / (32 * p.KB), nqt = (S + 31) / 32;
  p.ch = nqt;
  if (static_cast<int64_t>(nkg) * BHkv < 2 * static_cast<int64_t>(device_cus())) {
    const char* e = std::getenv("HYDRA_ATTN_BWD_CHUNK");
    p.ch = std::max(1, std::min({nqt, 16, e ? std::atoi(e) : 16}));
  }
  p.nwg = 0;
  for (int kg = 0; kg < nkg; ++kg) p.nwg += ((causal ? nqt - p.KB * kg : nqt) + p.ch - 1) / p.ch;
  p.maxch = (nqt + p.ch - 1) / p.ch;
  p.part_bytes = p.maxch > 1 ? static_cast<size_t>(BHkv) * nkg * p.maxch * p.KB * 32 * hd * 2 * 4 : 0;
  return p;
}

// A side stream per device (default priority, non-blocking) with a fork and
// a join event.  fork() makes the side stream wait for everything queued on
// the caller's stream so far; finish() makes the caller's stream wait for
// everything queued on the side stream since.  The lock, held from fork to
// finish, serialises the sequences of concurrent callers on one device.
// Inside a graph capture the pair is the usual cross-stream fork/join; the
// stream and events are only created outside one (a capture's first call
// runs on the caller's stream alone).
struct SideStream {
  std::unique_lock<std::mutex> lock;
  hipStream_t stream = nullptr, main = nullptr;
  hipEvent_t join = nullptr;

  bool fork(hipStream_t st) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static hipStream_t streams[kMaxDevices] = {};
    static hipEvent_t forks[kMaxDevices] = {}, joins[kMaxDevices] = {};
    // Only for a stream of the current device (the side stream lives there).
    int dev = 0;
    hipDevice_t sdev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices ||
        hipStreamGetDevice(st, &sdev) != hipSuccess || sdev != dev)
      return false;
    lock = std::unique_lock<std::mutex>(mu);
    if (streams[dev] == nullptr) {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
      hipStream_t s = nullptr;
      hipEvent_t f = nullptr, j = nullptr;
      if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return false;
      if (hipEventCreateWithFlags(&f, hipEventDisableTiming) != hipSuccess ||
          hipEventCreateWithFlags(&j, hipEventDisableTiming) != hipSuccess) {
        if (f) (void)hipEventDestroy(f);
        (void)hipStreamDestroy(s);
        return false;
      }
      streams[dev] = s;
      forks[dev] = f;
      joins[dev] = j;
    }
    if (hipEventRecord(forks[dev], st) != hipSuccess ||
        hipStreamWaitEvent(streams[dev], forks[dev], 0) != hipSuccess)
      return false;
    stream = streams[dev];
    join = joins[dev];
    main = st;
    return true;
  }
  int finish() {
    if (stream == nullptr) return HYDRA_OK;
    if (hipEventRecord(join, stream) != hipSuccess || hipStreamWaitEvent(main, join, 0) != hipSuccess)
      return fail(HYDRA_ERR_LAUNCH, "attn_bwd: joining the side stream failed");
    stream = nullptr;
    return HYDRA_OK;
  }
};

template <int HD, bool CAUSAL>
int launch_mfma(const BwdArgs& a, const float* dvec, const float* lse2, float* part) {
  const float sl2 = a.scale * kLog2e;
  const int BHkv = a.B * a.Hkv, G = a.Hq / a.Hkv;
  const bf16* q = static_cast<const bf16*>(a.q);
  const bf16* k = static_cast<const bf16*>(a.k);
  const bf16* v = static_cast<const bf16*>(a.v);
  const bf16* d = static_cast<const bf16*>(a.dout);
  // dQ needs only the row-dot's outputs, so it runs on a side stream,
  // concurrently with dK/dV: the two launches' causal tails (CUs whose
  // workgroups are done while others still walk the longest key ranges)
  // take each other's workgroups.
  SideStream side;
  const hipStream_t dq_st = side.fork(a.st) ? side.stream : a.st;
  auto launch_dq = [&]() {
    // An item is NW query tasks (32 query rows of one head) sharing each
    // staged K/V tile.
    constexpr int NW = kDqWaves;
    const int ntasks = ((a.S + 31) / 32) * G;
    const int items = (ntasks + NW - 1) / NW;
    attn_bwd_dq_kernel<HD, CAUSAL, NW><<<dim3(static_cast<unsigned>(items * BHkv)), 64 * NW, 0, dq_st>>>(
        q, k, v, d, dvec, lse2, static_cast<bf16*>(a.dq), a.Hq, a.Hkv, a.S, G, ntasks, items,
        a.qs[0], a.qs[1], a.qs[2], a.ks[0], a.ks[1], a.ks[2], a.vs[0], a.vs[1], a.vs[2], a.dos[0],
        a.dos[1], a.dos[2], a.dqs[0], a.dqs[1], a.dqs[2], sl2, a.scale);
    return check_launch("attn_bwd: dq");
  };
  auto launch_dkdv = [&]() -> int {
    const DkdvPlan pl = plan_dkdv(HD, a.S, G, BHkv, CAUSAL);
    const dim3 grid(static_cast<unsigned>(pl.nwg * BHkv));
#define HYDRA_DKDV(KBV, HGV)                                                                     \
  attn_bwd_dkdv_kernel<HD, CAUSAL, KBV, HGV><<<grid, 64 * KBV * HGV, 0, a.st>>>(                 \
      q, k, v, d, dvec, lse2, static_cast<bf16*>(a.dk), static_cast<bf16*>(a.dv), part, a.Hq,   \
      a.Hkv, a.S, G, pl.nwg, pl.ch, pl.maxch, a.qs[0], a.qs[1], a.qs[2], a.ks[0], a.ks[1],      \
      a.ks[2], a.vs[0], a.vs[1], a.vs[2], a.dos[0], a.dos[1], a.dos[2], a.dks[0], a.dks[1],     \
      a.dks[2], a.dvs[0], a.dvs[1], a.dvs[2], sl2, a.scale);                                     \
  if (int rc = check_launch("attn_bwd: dkdv")) return rc;                                       \
  if (pl.maxch > 1) {                                                                            \
    attn_bwd_dkdv_reduce_kernel<HD, CAUSAL, KBV>                                                 \
        <<<dim3(static_cast<unsigned>((a.S * (HD / 4) + 255) / 256),                             \
                static_cast<unsigned>(std::min(BHkv, 65535)),                                    \
                static_cast<unsigned>((BHkv + 65534) / 65535)), 256, 0, a.st>>>(                 \
            part, static_cast<bf16*>(a.dk), static_cast<bf16*>(a.dv), BHkv, a.Hkv, a.S, pl.ch,   \
            pl.maxch, a.dks[0], a.dks[1], a.dks[2], a.dvs[0], a.dvs[1], a.dvs[2], a.scale);      \
    if (int rc = check_launch("attn_bwd: dkdv reduce")) return rc;                              \
  }
    if constexpr (HD <= 64) {
      if (pl.HG == 2) {
        HYDRA_DKDV(4, 2)
      }
    }
    if (pl.HG == 1) {
      HYDRA_DKDV(4, 1)
    }
#undef HYDRA_DKDV
    return HYDRA_OK;
  };
  // every path joins the side stream back before returning
  int rc = launch_dkdv();
  if (rc == HYDRA_OK) rc = launch_dq();
  const int rj = side.finish();
  return rc != HYDRA_OK ? rc : rj;
}

template <typename T, int MAXD, bool CAUSAL, int MASK>
int launch_generic(const BwdArgs& a, const float* dvec, const float* lse2) {
  const float sl2 = a.scale * kLog2e;
  const T* q = static_cast<const T*>(a.q);
  const T* k = static_cast<const T*>(a.k);
  const T* v = static_cast<const T*>(a.v);
  const T* d = static_cast<const T*>(a.dout);
  const int64_t qrows = static_cast<int64_t>(a.B) * a.Hq * a.S;
  const int64_t krows = static_cast<int64_t>(a.B) * a.Hkv * a.S;
  attn_bwd_generic_dkdv_kernel<T, MAXD, CAUSAL, MASK>
      <<<dim3(static_cast<unsigned>((krows + 127) / 128)), 128, 0, a.st>>>(
          q, k, v, d, dvec, lse2, a.kmask, static_cast<T*>(a.dk), static_cast<T*>(a.dv), krows, a.Hq,
          a.Hkv, a.S, a.hd, a.qs[0], a.qs[1], a.qs[2], a.ks[0], a.ks[1], a.ks[2], a.vs[0],
          a.vs[1], a.vs[2], a.dos[0], a.dos[1], a.dos[2], a.dks[0], a.dks[1], a.dks[2],
          a.dvs[0], a.dvs[1], a.dvs[2], sl2, a.scale);
  if (int rc = check_launch("attn_bwd: generic dkdv")) return rc;
  attn_bwd_generic_dq_kernel<T, MAXD, CAUSAL, MASK>
      <<<dim3(static_cast<unsigned>((qrows + 127) / 128)), 128, 0, a.st>>>(
          q, k, v, d, dvec, lse2, a.kmask, static_cast<T*>(a.dq), qrows, a.Hq, a.Hkv, a.S, a.hd,
          a.qs[0], a.qs[1], a.qs[2], a.ks[0], a.ks[1], a.ks[2], a.vs[0], a.vs[1], a.vs[2],
          a.dos[0], a.dos[1], a.dos[2], a.dqs[0], a.dqs[1], a.dqs[2], sl2, a.scale);
  return check_launch("attn_bwd: generic dq");
}

template <typename T, bool CAUSAL, int MASK>
int launch_generic_d(const BwdArgs& a, const float* dvec, const float* lse2) {
  if (a.hd <= 32) return launch_generic<T, 32, CAUSAL, MASK>(a, dvec, lse2);
  if (a.hd <= 64) return launch_generic<T, 64, CAUSAL, MASK>(a, dvec, lse2);
  if (a.hd <= 128) return launch_generic<T, 128, CAUSAL, MASK>(a, dvec, lse2);
  return launch_generic<T, 256, CAUSAL, MASK>(a, dvec, lse2);
}

template <typename T>
int run_generic(const BwdArgs& a, float* dvec, float* lse2) {
  if (int rc = launch_rowdot<T>(a, dvec, lse2)) return rc;
  if (a.mask_mode == HYDRA_MASK_REFERENCE_SDPA) return launch_generic_d<T, true, 2>(a, dvec, lse2);
  if (a.mask_mode == HYDRA_MASK_KEY_PADDING)
    return a.causal ? launch_generic_d<T, true, 1>(a, dvec, lse2) : launch_generic_d<T, false, 1>(a, dvec, lse2);
  return a.causal ? launch_generic_d<T, true, 0>(a, dvec, lse2)
                  : launch_generic_d<T, false, 0>(a, dvec, lse2);
}

template <int HD>
int run_mfma(const BwdArgs& a, float* dvec, float* lse2, float* part) {
  if (int rc = launch_rowdot<bf16>(a, dvec, lse2)) return rc;
  return a.causal ? launch_mfma<HD, true>(a, dvec, lse2, part)
                  : launch_mfma<HD, false>(a, dvec, lse2, part);
}

}  // namespace
}  // namespace hydra

using namespace hydra;

// hydra_attn_bwd, or with need != nullptr the scratch bytes it would take
// (no pointers needed; assumed 16-byte aligned, so the answer covers the
// MFMA path whenever the shapes allow it).
static int attn_bwd_impl(const void* q, const void* k, const void* v, const void* o,
                         const void* grad_o, const float* lse, void* grad_q, void* grad_k,
                         void* grad_v, int64_t B, int64_t Hq, int64_t Hkv, int64_t S,
                         int64_t hd, const int64_t* qs, const int64_t* ks,
                         const int64_t* vs, const int64_t* os, const int64_t* gos,
                         const int64_t* gqs, const int64_t* gks, const int64_t* gvs,
                         const uint8_t* key_mask, int mask_mode, int causal, float scale,
                         int dtype, void* workspace, int64_t workspace_bytes, size_t* need,
                         void* stream) {
  if (need) *need = 0;
  HYDRA_REQUIRE(workspace_bytes >= 0, "attn_bwd: negative workspace size");
  HYDRA_REQUIRE(mask_mode >= HYDRA_MASK_NONE && mask_mode <= HYDRA_MASK_REFERENCE_SDPA,
                "attn_bwd: unknown mask mode");
  HYDRA_REQUIRE(mask_mode == HYDRA_MASK_NONE || key_mask != nullptr || need,
                "attn_bwd: mask mode needs key_mask");
  HYDRA_REQUIRE(mask_mode != HYDRA_MASK_REFERENCE_SDPA || causal,
                "attn_bwd: the reference-SDPA mask mode is defined with causal=1");
  HYDRA_REQUIRE(B >= 0 && S >= 0 && Hq >= 1 && Hkv >= 1 && hd >= 1, "attn_bwd: bad size");
  HYDRA_REQUIRE(Hq % Hkv == 0, "attn_bwd: n_heads must be a multiple of n_kv_heads");
  HYDRA_REQUIRE(qs && ks && vs && os && gos && gqs && gks && gvs, "attn_bwd: null stride array");
  HYDRA_REQUIRE(qs[3] == 1 && ks[3] == 1 && vs[3] == 1 && os[3] == 1 && gos[3] == 1 &&
                    gqs[3] == 1 && gks[3] == 1 && gvs[3] == 1,
                "attn_bwd: every tensor needs unit stride along head_dim");
  HYDRA_REQUIRE(hd <= 256, "attn_bwd: head_dim must be <= 256");
  HYDRA_REQUIRE(dtype == HYDRA_F32 || dtype == HYDRA_BF16 || dtype == HYDRA_F16,
                "attn_bwd: unknown dtype");
  if (B * S == 0) return HYDRA_OK;
  HYDRA_REQUIRE(need || (q && k && v && o && grad_o && lse && grad_q && grad_k && grad_v),
                "attn_bwd: null pointer");
  HYDRA_REQUIRE(S < (int64_t(1) << 30) && B * Hq * S < (int64_t(1) << 31),
                "attn_bwd: problem too large");
  auto st = static_cast<hipStream_t>(stream);
  const int64_t rows = B * Hq * S;
  const BwdArgs a{q, k, v, o, grad_o, lse, grad_q, grad_k, grad_v, static_cast<int>(B),
                  static_cast<int>(Hq), static_cast<int>(Hkv), static_cast<int>(S),
                  static_cast<int>(hd), qs, ks, vs, os, gos, gqs, gks, gvs, causal != 0, scale,
                  st, mask_mode != HYDRA_MASK_NONE ? key_mask : nullptr, mask_mode};
  // a key mask takes the VALU kernels
  bool mfma_ok = dtype == HYDRA_BF16 && (hd == 32 || hd == 64 || hd == 128) && mask_mode == HYDRA_MASK_NONE;
  // Tiles are addressed with 32-bit byte offsets within one head's rows
  // (up to 64 rows past S).
  for (const int64_t* s : {qs, ks, vs, gos, gqs, gks, gvs})
    mfma_ok = mfma_ok && s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0 && s[2] >= hd &&
              (S + 64) * s[2] * 2 < (int64_t(1) << 31);
  if (!need)
    for (const void* p : {q, k, v, grad_o, static_cast<const void*>(grad_q),
                          static_cast<const void*>(grad_k), static_cast<const void*>(grad_v)})
      mfma_ok = mfma_ok && aligned16(p);
  // Workspace: D and lse2 per query row, then the dK/dV chunk partials.
  const size_t rows_bytes = (static_cast<size_t>(rows) * 2 * sizeof(float) + 255) & ~size_t(255);
  const size_t part_bytes =
      mfma_ok ? plan_dkdv(static_cast<int>(hd), static_cast<int>(S), static_cast<int>(Hq / Hkv),
                          static_cast<int>(B * Hkv), causal != 0).part_bytes
              : 0;
  if (need) {
    *need = rows_bytes + part_bytes;
    return HYDRA_OK;
  }
  if (workspace == nullptr || static_cast<size_t>(workspace_bytes) < rows_bytes + part_bytes)
    return fail(HYDRA_ERR_ARG, "attn_bwd: workspace of " + std::to_string(rows_bytes + part_bytes) +
                                   " bytes required (hydra_attn_bwd_workspace)");
  void* ws = workspace;
  float* dvec = static_cast<float*>(ws);
  float* lse2 = dvec + rows;
  float* part = reinterpret_cast<float*>(static_cast<char*>(ws) + rows_bytes);
  if (mfma_ok) {
    switch (hd) {
      case 32: return run_mfma<32>(a, dvec, lse2, part);
      case 64: return run_mfma<64>(a, dvec, lse2, part);
      default: return run_mfma<128>(a, dvec, lse2, part);
    }
  }
  switch (dtype) {
    case HYDRA_F32: return run_generic<float>(a, dvec, lse2);
    case HYDRA_BF16: return run_generic<bf16>(a, dvec, lse2);
    default: return run_generic<f16>(a, dvec, lse2);
  }
}

extern "C" int hydra_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                              const void* grad_o, const float* lse, void* grad_q, void* grad_k,
                              void* grad_v, int64_t B, int64_t Hq, int64_t Hkv, int64_t S,
                              int64_t hd, const int64_t* qs, const int64_t* ks,
                              const int64_t* vs, const int64_t* os, const int64_t* gos,
                              const int64_t* gqs, const int64_t* gks, const int64_t* gvs,
                              const uint8_t* key_mask, int mask_mode, int causal, float scale,
                              int dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  return attn_bwd_impl(q, k, v, o, grad_o, lse, grad_q, grad_k, grad_v, B, Hq, Hkv, S, hd, qs, ks, vs, os,
                       gos, gqs, gks, gvs, key_mask, mask_mode, causal, scale, dtype, workspace,
                       workspace_bytes, nullptr, stream);
}

extern "C" int hydra_attn_bwd_workspace(int64_t B, int64_t Hq, int64_t Hkv, int64_t S, int64_t hd,
                                        const int64_t* qs, const int64_t* ks, const int64_t* vs,
                                        const int64_t* os, const int64_t* gos, const int64_t* gqs,
                                        const int64_t* gks, const int64_t* gvs, int mask_mode,
                                        int causal, int dtype, int64_t* bytes) {
  HYDRA_REQUIRE(bytes != nullptr, "attn_bwd_workspace: null result pointer");
  size_t need = 0;
  const int rc = attn_bwd_impl(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, B,
                               Hq, Hkv, S, hd, qs, ks, vs, os, gos, gqs, gks, gvs, nullptr, mask_mode, causal,
                               1.f, dtype, nullptr, 0, &need, nullptr);
  *bytes = static_cast<int64_t>(need);
  return rc;
}
