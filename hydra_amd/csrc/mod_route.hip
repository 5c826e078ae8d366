// Mixture-of-Depths hard routing on gfx950: per-row top-k select with
// lowest-index tie-breaking, row gather, and in-place weighted residual
// scatter (hydra/routing/mixture_of_depths.py:159-216,
// hydra/model/framework/blocks.py:243-269).
//
// Top-k: each score becomes a 64-bit composite key
//   (~order_preserving_u32(score) << 32) | index
// so that an ascending sort gives value-descending order with ties resolved
// by ascending index, i.e. the order of a stable descending sort.  Rows of
// up to 8192 keys take the bucket kernel (a counting sort over the keys' top
// bits in LDS, several workgroups per row; rows whose bins degenerate fall
// back to a bitonic sort in LDS by one workgroup); longer rows a device-wide
// radix sort in global memory (mod_topk_large.hip).  The ascending
// index list comes from a bitmap of the selection and a block prefix count.
#include "common.h"
#include "mod_keys.h"

#include <cstdlib>
#include <type_traits>

namespace hydra {

constexpr int kTopkThreads = 1024;

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Bitonic sort of P = EPT * kTopkThreads keys, ascending.  Thread t holds
// keys [EPT*t, EPT*t + EPT) in registers: strides below EPT are compared in
// the thread, strides below 64*EPT by exchanging with lane ^ (stride/EPT),
// and only the larger strides go through LDS (one barrier each).
template <int EPT>
__device__ __forceinline__ void bitonic_sort(uint64_t (&v)[EPT], uint64_t* lds, int tid) {
  constexpr int P = EPT * kTopkThreads;
  constexpr int WSPAN = 64 * EPT;  // keys held by one wave
  const int i0 = EPT * tid;
  // Merge steps with strides < WSPAN, for one `size`, entirely in registers.
  auto reg_merge = [&](int size, int top) {
    for (int stride = top; stride > 0; stride >>= 1) {
      if (stride >= EPT) {
        const int m = stride / EPT;
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
          const int i = i0 + j;
          const uint64_t o = shfl_xor_u64(v[j], m);
          const bool up = (i & size) == 0;
          const bool lo = (i & stride) == 0;
          const uint64_t mn = v[j] < o ? v[j] : o, mx = v[j] < o ? o : v[j];
          v[j] = (lo == up) ? mn : mx;
        }
      } else {
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
          if ((j & stride) == 0) {
            const int i = i0 + j;
            const bool up = (i & size) == 0;
            const uint64_t a = v[j], b = v[j + stride];
            const bool sw = (a > b) == up;
            v[j] = sw ? b : a;
            v[j + stride] = sw ? a : b;
          }
        }
      }
    }
  };
  for (int size = 2; size <= P; size <<= 1) {
    int stride = size >> 1;
    if (stride >= WSPAN) {
      // cross-wave strides in LDS
#pragma unroll
      for (int j = 0; j < EPT; ++j) lds[i0 + j] = v[j];
      __syncthreads();
      for (; stride >= WSPAN; stride >>= 1) {
        for (int t = tid; t < P / 2; t += kTopkThreads) {
          const int lo = 2 * t - (t & (stride - 1));
          const int hi = lo + stride;
          const bool up = (lo & size) == 0;
          const uint64_t a = lds[lo], b = lds[hi];
          if ((a > b) == up) {
            lds[lo] = b;
            lds[hi] = a;
          }
        }
        __syncthreads();
      }
#pragma unroll
      for (int j = 0; j < EPT; ++j) v[j] = lds[i0 + j];
      __syncthreads();  // everyone has read before the next size rewrites LDS
    }
    reg_merge(size, stride);
  }
#pragma unroll
  for (int j = 0; j < EPT; ++j) lds[i0 + j] = v[j];
  __syncthreads();
}

template <typename S, int EPT>
__global__ __launch_bounds__(kTopkThreads) void mod_topk_kernel(
    const S* __restrict__ scores, int L, int64_t s_rs, int k,
    int64_t* __restrict__ idx_desc, int64_t* __restrict__ idx_sorted,
    void* __restrict__ mask, int mask_dtype) {
  constexpr int P = EPT * kTopkThreads;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  uint64_t* keys = reinterpret_cast<uint64_t*>(smem);
  uint32_t* bits = reinterpret_cast<uint32_t*>(smem + sizeof(uint64_t) * P);
  __shared__ int wave_tot[kTopkThreads / 64];

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const S* sr = scores + static_cast<int64_t>(row) * s_rs;

  uint64_t v[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int i = EPT * tid + j;
    uint64_t key = ~uint64_t(0);
    if (i < L) {
      const uint32_t desc = ~score_key_asc(to_f32(sr[i]));
      key = (static_cast<uint64_t>(desc) << 32) | static_cast<uint32_t>(i);
    }
    v[j] = key;
  }
  const int nwords = (L + 31) / 32;
  for (int i = tid; i < nwords; i += kTopkThreads) bits[i] = 0u;
  bitonic_sort<EPT>(v, keys, tid);

  int64_t* drow = idx_desc ? idx_desc + static_cast<int64_t>(row) * k : nullptr;
  for (int j = tid; j < k; j += kTopkThreads) {
    const uint32_t i = static_cast<uint32_t>(keys[j] & 0xffffffffu);
    if (drow) drow[j] = static_cast<int64_t>(i);
    atomicOr(&bits[i >> 5], 1u << (i & 31));
  }
  __syncthreads();

  if (mask) {
    const int64_t mrow = static_cast<int64_t>(row) * L;
    for (int i = tid; i < L; i += kTopkThreads) {
      const float v = (bits[i >> 5] >> (i & 31)) & 1u ? 1.f : 0.f;
      switch (mask_dtype) {
        case HYDRA_F32: static_cast<float*>(mask)[mrow + i] = v; break;
        case HYDRA_BF16: static_cast<bf16*>(mask)[mrow + i] = from_f32<bf16>(v); break;
        default: static_cast<f16*>(mask)[mrow + i] = from_f32<f16>(v); break;
      }
    }
  }
  if (!idx_sorted) return;

  // Ascending indices: thread t owns words [t*wpt, (t+1)*wpt) of the bitmap;
  // an exclusive prefix over the per-thread popcounts gives each thread its
  // output offset.
  const int wpt = (nwords + kTopkThreads - 1) / kTopkThreads;
  const int w0 = tid * wpt;
  int cnt = 0;
  for (int w = w0; w < w0 + wpt && w < nwords; ++w) cnt += __popc(bits[w]);
  const int lane = tid & 63, wave = tid >> 6;
  const int incl = wave_incl_sum(cnt);
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += wave_tot[w];
  int pos = base + incl - cnt;
  int64_t* orow = idx_sorted + static_cast<int64_t>(row) * k;
  for (int w = w0; w < w0 + wpt && w < nwords; ++w) {
    uint32_t m = bits[w];
    while (m) {
      const int b = __ffs(m) - 1;
      m &= m - 1;
      if (pos < k) orow[pos] = static_cast<int64_t>(w * 32 + b);
      ++pos;
    }
  }
}

// ---- bucketed top-k (rows of up to kBucketMaxL keys) ---------------------
// R workgroups per row (R = ceil(L / 1024)), each running:
//  1. keys: desc(score) = ~score_key_asc(score) (ascending desc <-> value-
//     descending, NaN first, -0.0 == +0.0); histogram of its top kBinBits
//     bits in LDS (atomic adds; each key keeps its slot within its bin);
//  2. exclusive scan of the histogram -> the first position of every bin in
//     the value-descending order; whether any bin is over kBucketMaxBin, and
//     the bin holding position k-1 (the threshold bin);
//  3. every key written to its bin's segment as the 64-bit composite
//     (desc << 32) | index, so keys[] is in bin order;
//  4. the selection bitmap of the keys below the threshold bin, and of the
//     threshold bin's keys of rank < k (see 5);
//  5. the rank of a key = first position of its bin + the keys of its bin
//     with a smaller composite (a larger score, or an equal score at a lower
//     index) -- exact, the order of a stable descending sort.  Keys below the
//     threshold bin are selected, keys above are not, keys in it are
//     selected when their rank is < k; the workgroup ranks the keys of the
//     bins up to the threshold bin that start at positions [1024 part,
//     1024 part + 1024) of keys[] and writes idx_desc[rank] = index;
//  6. prefix counts over the bitmap's words give the mask and the ascending
//     list entries of the workgroup's part of the row.
// Steps 1-4 are repeated by each of a row's workgroups (cheap); the ranks,
// the expensive part, are split between them.  Bins are small for real
// score distributions (tens of keys for N(0, 1) scores at L = 4096); when the
// largest bin exceeds kBucketMaxBin keys (e.g. many equal scores) the row's
// first workgroup sorts the whole row with the bitonic sort instead and the
// others leave, so the cost stays bounded.
constexpr int kBinBits = 14;
constexpr int kBins = 1 << kBinBits;
// Bins live in LDS with 4 pad words after every 16 (kBinWords in all), so
// the scan's per-thread runs of 16 bins (16-byte reads, 80 bytes apart) fall
// in distinct banks.
constexpr int kBinWords = kBins + kBins / 4;
__device__ __forceinline__ uint32_t bin_slot(uint32_t b) { return b + 4 * (b >> 4); }
constexpr int kBucketMaxL = 8192;
constexpr int kLdsMaxL = 16384;  // longest row the bitonic kernel sorts in LDS
constexpr int kBucketMaxBin = 512;
constexpr int kKeyPad = 8;  // all-ones keys after the row, read by seg_rank

// Rank of composite `me` among the row's keys, given its bin's segment
// [b0, b1) of the bin-ordered keys[]: b0 + the segment's keys below `me`.
// The reads start at b0 rounded down to an even position (16-byte aligned;
// the lanes of a wave that rank different bins then spread over the LDS
// banks) and run in rounds of 8 keys past b1: the key before b0 belongs to
// a lower bin (below `me`, so it counts b0 - s) and those at or after b1 to
// higher bins or the all-ones padding after the row (never below `me`), so
// the rank is s + the count.
__device__ __forceinline__ int seg_rank(const uint64_t* keys, int b0, int b1, uint64_t me) {
  const int s = b0 & ~1;
  int r = s;
  for (int j = s; j < b1; j += 8) {
    const uint4* q = reinterpret_cast<const uint4*>(keys + j);
    uint4 w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) w[u] = q[u];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint64_t a = (static_cast<uint64_t>(w[u].y) << 32) | w[u].x;
      const uint64_t c = (static_cast<uint64_t>(w[u].w) << 32) | w[u].z;
      r += (a < me ? 1 : 0) + (c < me ? 1 : 0);
    }
  }
  return r;
}

template <typename S, int EPT>
__global__ __launch_bounds__(kTopkThreads) void mod_topk_bucket_kernel(
    const S* __restrict__ scores, int L, int64_t s_rs, int k, int R,
    int64_t* __restrict__ idx_desc, int64_t* __restrict__ idx_sorted,
    void* __restrict__ mask, int mask_dtype) {
  constexpr int P = EPT * kTopkThreads;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  uint64_t* keys = reinterpret_cast<uint64_t*>(smem);                                      // [P + 8]
  uint32_t* hist = reinterpret_cast<uint32_t*>(smem + sizeof(uint64_t) * (P + kKeyPad));  // [kBinWords]
  uint32_t* bits = hist + kBinWords;                                                       // [L/32] selection
  uint32_t* wpre = bits + P / 32;                                                          // [L/32] word prefixes
  // per wave: bin count | (any bin > kBucketMaxBin) << 16; then popcounts
  __shared__ __align__(16) int wave_tot[kTopkThreads / 64];
  __shared__ __align__(16) int wave_pc[kTopkThreads / 64];
  __shared__ int thr[2];  // threshold bin, its first position

  const int row = blockIdx.x / R, part = blockIdx.x - row * R;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const S* sr = scores + static_cast<int64_t>(row) * s_rs;
  // the row's scores load while the bins clear; element e of this thread
  // is i = tid + 1024 e
  S raw[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int i = tid + kTopkThreads * e;
    raw[e] = i < L ? sr[i] : S();
  }
  static_assert(kBinWords % (4 * kTopkThreads) == 0, "bins clear in whole 16-byte rounds");
#pragma unroll
  for (int i = tid; i < kBinWords / 4; i += kTopkThreads) reinterpret_cast<uint4*>(hist)[i] = make_uint4(0u, 0u, 0u, 0u);
  const int nwords = (L + 31) / 32;
  for (int i = tid; i < nwords; i += kTopkThreads) bits[i] = 0u;
  __syncthreads();

  // 1. histogram of the keys (each key keeps its slot within its bin)
  uint32_t dk[EPT], slot[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const int i = tid + kTopkThreads * e;
    dk[e] = i < L ? ~score_key_asc(to_f32(raw[e])) : 0u;
    slot[e] = i < L ? atomicAdd(&hist[bin_slot(dk[e] >> (32 - kBinBits))], 1u) : 0u;
  }
  __syncthreads();

  // 2. exclusive scan of the bins: thread t owns bins [16 t, 16 t + 16)
  constexpr int BPT = kBins / kTopkThreads;
  static_assert(BPT == 16, "a thread's bins are one padded run of 16");
  uint32_t hv[BPT];
  uint4* hrun = reinterpret_cast<uint4*>(hist + 20 * tid);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 w = hrun[q];
    hv[4 * q] = w.x; hv[4 * q + 1] = w.y; hv[4 * q + 2] = w.z; hv[4 * q + 3] = w.w;
  }
  int cnt = 0;
  bool big = false;
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    cnt += static_cast<int>(hv[j]);
    big |= hv[j] > static_cast<uint32_t>(kBucketMaxBin);
  }
  const int incl = wave_incl_sum(cnt);
  const bool wbig = __ballot(big) != 0;
  if (lane == 63) wave_tot[wave] = incl | (wbig ? 1 << 16 : 0);
  __syncthreads();
  int base = 0, nbig = 0;
#pragma unroll
  for (int q = 0; q < kTopkThreads / 256; ++q) {
    const int4 t = reinterpret_cast<const int4*>(wave_tot)[q];
    const int tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      base += 4 * q + u < wave ? (tv[u] & 0xffff) : 0;
      nbig += tv[u] >> 16;
    }
  }
  if (nbig) {
    // Degenerate bins: the row's first workgroup sorts the whole row (ties
    // by index, as above) and writes every output; the others leave.
    if (part != 0) return;
    uint64_t v[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      const int i = EPT * tid + j;
      v[j] = ~uint64_t(0);
      if (i < L) v[j] = (static_cast<uint64_t>(~score_key_asc(to_f32(sr[i]))) << 32) | static_cast<uint32_t>(i);
    }
    bitonic_sort<EPT>(v, keys, tid);  // leaves the sorted row in keys[]
    for (int j = tid; j < k; j += kTopkThreads) {
      const uint32_t i = static_cast<uint32_t>(keys[j] & 0xffffffffu);
      if (idx_desc) idx_desc[static_cast<int64_t>(row) * k + j] = static_cast<int64_t>(i);
      atomicOr(&bits[i >> 5], 1u << (i & 31));
    }
  } else {
    int pos = base + incl - cnt;
    if (pos <= k - 1 && k - 1 < pos + cnt) {  // exactly one thread's bins hold position k-1
      // the threshold bin is the first whose end passes k-1
      int q = pos, jt = 0, pt = pos;
#pragma unroll
      for (int j = 0; j < BPT; ++j) {
        q += static_cast<int>(hv[j]);
        const bool before = q <= k - 1;
        jt += before ? 1 : 0;
        pt = before ? q : pt;
      }
      thr[0] = tid * BPT + jt;
      thr[1] = pt;
    }
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      const int c = static_cast<int>(hv[j]);
      hv[j] = static_cast<uint32_t>(pos);  // first position of the bin
      pos += c;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) hrun[q] = make_uint4(hv[4 * q], hv[4 * q + 1], hv[4 * q + 2], hv[4 * q + 3]);
    if (tid < kKeyPad) keys[L + tid] = ~uint64_t(0);  // padding read by seg_rank
    __syncthreads();
    // 3. composites into their bins' segments
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int i = tid + kTopkThreads * e;
      if (i < L)
        keys[hist[bin_slot(dk[e] >> (32 - kBinBits))] + slot[e]] =
            (static_cast<uint64_t>(dk[e]) << 32) | static_cast<uint32_t>(i);
    }
    __syncthreads();
    const uint32_t tb = static_cast<uint32_t>(thr[0]);
    const int tb0 = thr[1];
    const int tb1 = tb + 1 < kBins ? static_cast<int>(hist[bin_slot(tb + 1)]) : L;
    // 4. the selection bitmap below the threshold bin: a wave's 64
    // consecutive keys -> two bitmap words by ballot, OR-ed in by one lane
    // (the threshold bin's bits below may share the words)
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int i = tid + kTopkThreads * e;
      const uint64_t sel = __ballot(i < L && (dk[e] >> (32 - kBinBits)) < tb);
      const int w0 = (kTopkThreads * e + 64 * wave) >> 5;
      if (lane == 0 && w0 < nwords && static_cast<uint32_t>(sel)) atomicOr(&bits[w0], static_cast<uint32_t>(sel));
      if (lane == 0 && w0 + 1 < nwords && static_cast<uint32_t>(sel >> 32))
        atomicOr(&bits[w0 + 1], static_cast<uint32_t>(sel >> 32));
    }
    // 5. the threshold bin's keys of rank < k complete the bitmap
    for (int p = tb0 + tid; p < tb1; p += kTopkThreads) {
      const uint64_t me = keys[p];
      if (seg_rank(keys, tb0, tb1, me) < k) {
        const uint32_t i = static_cast<uint32_t>(me & 0xffffffffu);
        atomicOr(&bits[i >> 5], 1u << (i & 31));
      }
    }
    // 6. ranks in bin order.  The slot order inside a bin differs between
    // the row's workgroups, so the split between them follows bins: this
    // part ranks the bins that start among its positions [1024 part,
    // 1024 part + 1024), up to the end of the last of them (a bin holds at
    // most kBucketMaxBin keys) or of the threshold bin.  A wave's 64
    // positions share a few bins, so the segment reads are mostly broadcasts.
    if (idx_desc) {
      const int plo = kTopkThreads * part;
      int phi = plo + kTopkThreads;
      if (phi < tb1) {
        const uint32_t bl = static_cast<uint32_t>(keys[phi - 1] >> (64 - kBinBits));
        phi = bl == tb ? tb1 : static_cast<int>(hist[bin_slot(bl + 1)]);
      }
      phi = min(phi, tb1);
      for (int p = plo + tid; p < phi; p += kTopkThreads) {
        const uint64_t me = keys[p];
        const uint32_t b = static_cast<uint32_t>(me >> (64 - kBinBits));
        const int b0 = static_cast<int>(hist[bin_slot(b)]);
        if (b0 < plo) continue;  // the previous part's bin
        const int b1 = b == tb ? tb1 : static_cast<int>(hist[bin_slot(b + 1)]);
        const int r = seg_rank(keys, b0, b1, me);
        if (r < k) idx_desc[static_cast<int64_t>(row) * k + r] = static_cast<int64_t>(me & 0xffffffffu);
      }
    }
  }
  __syncthreads();

  // mask and ascending list of this part: elements [1024 part, 1024 part + 1024)
  const int i0 = kTopkThreads * part;
  if (mask) {
    const int64_t mrow = static_cast<int64_t>(row) * L;
    const int hi = nbig ? L : min(L, i0 + kTopkThreads);
    for (int i = (nbig ? 0 : i0) + tid; i < hi; i += kTopkThreads) {
      const float v = (bits[i >> 5] >> (i & 31)) & 1u ? 1.f : 0.f;
      switch (mask_dtype) {
        case HYDRA_F32: static_cast<float*>(mask)[mrow + i] = v; break;
        case HYDRA_BF16: static_cast<bf16*>(mask)[mrow + i] = from_f32<bf16>(v); break;
        default: static_cast<f16*>(mask)[mrow + i] = from_f32<f16>(v); break;
      }
    }
  }
  if (!idx_sorted) return;
  // word prefixes: exclusive scan of the popcounts of the row's words
  // (nwords <= 256 < 1024: thread t owns word t)
  const int pc = tid < nwords ? __popc(bits[tid]) : 0;
  const int pincl = wave_incl_sum(pc);
  if (lane == 63) wave_pc[wave] = pincl;
  __syncthreads();
  int pbase = 0;
#pragma unroll
  for (int q = 0; q < kTopkThreads / 256; ++q) {
    const int4 t = reinterpret_cast<const int4*>(wave_pc)[q];
    pbase += (4 * q < wave ? t.x : 0) + (4 * q + 1 < wave ? t.y : 0) + (4 * q + 2 < wave ? t.z : 0) +
             (4 * q + 3 < wave ? t.w : 0);
  }
  if (tid < nwords) wpre[tid] = static_cast<uint32_t>(pbase + pincl - pc);
  __syncthreads();
  int64_t* orow = idx_sorted + static_cast<int64_t>(row) * k;
  const int hi = nbig ? L : min(L, i0 + kTopkThreads);
  for (int i = (nbig ? 0 : i0) + tid; i < hi; i += kTopkThreads) {
    const uint32_t wbits = bits[i >> 5];
    if ((wbits >> (i & 31)) & 1u) {
      const int o = static_cast<int>(wpre[i >> 5]) + __popc(wbits & ((1u << (i & 31)) - 1u));
      if (o < k) orow[o] = static_cast<int64_t>(i);
    }
  }
}

// ---- row gather / scatter ------------------------------------------------
// One thread per 16-byte chunk of an output row; chunk -> (row, column) with
// 32-bit arithmetic (host checks the sizes).  An index outside [0, L) makes
// the row a no-op (gather writes zeros), so no access leaves the tensors.
template <typename T, int U>
__global__ __launch_bounds__(256) void mod_gather_kernel(
    const T* __restrict__ x, const int64_t* __restrict__ idx, T* __restrict__ xs,
    uint32_t total, uint32_t cpr, uint32_t k, int64_t L, int64_t x_bs, int64_t x_ls) {
  // U chunks per thread, 256 apart, all loads issued before the stores.
  constexpr int E = Vec<T>::N;
  const uint32_t base = blockIdx.x * (256 * U) + threadIdx.x;
  float f[U][E];
  uint32_t rr[U], cc[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t t = base + 256 * j;
    rr[j] = t / cpr;
    cc[j] = t - rr[j] * cpr;
    if (t >= total) continue;
    const uint32_t b = rr[j] / k;  // rr = b*k + j'
    const int64_t src = idx[rr[j]];
    if (src >= 0 && src < L) {
      load16<T, true>(x + b * x_bs + src * x_ls + cc[j] * E, f[j]);
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) f[j][e] = 0.f;
    }
  }
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t t = base + 256 * j;
    if (t < total) store16<T, true>(xs + static_cast<int64_t>(rr[j]) * cpr * E + cc[j] * E, f[j]);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void mod_gather_scalar_kernel(
    const T* __restrict__ x, const int64_t* __restrict__ idx, T* __restrict__ xs,
    int64_t total, int64_t D, int64_t k, int64_t L, int64_t x_bs, int64_t x_ls) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= total) return;
  const int64_t r = t / D, c = t - r * D;
  const int64_t b = r / k;
  const int64_t src = idx[r];
  xs[t] = (src >= 0 && src < L) ? x[b * x_bs + src * x_ls + c] : from_f32<T>(0.f);
}

template <typename T, int MODE, int U>
__global__ __launch_bounds__(256) void mod_scatter_kernel(
    T* __restrict__ out, const T* __restrict__ y, const int64_t* __restrict__ idx,
    const float* __restrict__ w, uint32_t total, uint32_t cpr, uint32_t k, int64_t L,
    int64_t o_bs, int64_t o_ls) {
  // U chunks per thread, 256 apart, all loads issued before the stores.
  constexpr int E = Vec<T>::N;
  const uint32_t base = blockIdx.x * (256 * U) + threadIdx.x;
  float yf[U][E], of[U][E];
  T* op[U];
  float wt[U];
#pragma unroll
  for (int j = 0; j < U; ++j) {
    const uint32_t t = base + 256 * j;
    op[j] = nullptr;
    if (t >= total) continue;
    const uint32_t r = t / cpr, c = t - r * cpr;
    const uint32_t b = r / k;
    const int64_t dst = idx[r];
    if (dst < 0 || dst >= L) continue;
    op[j] = out + b * o_bs + dst * o_ls + c * E;
    if (y) {
      load16<T, true>(y + static_cast<int64_t>(r) * cpr * E + c * E, yf[j]);
    } else {  // REPLACE without values: clear the rows
#pragma unroll
      for (int e = 0; e < E; ++e) yf[j][e] = 0.f;
    }
    if (MODE == HYDRA_SCATTER_ADD) {
      wt[j] = w ? w[r] : 1.f;
      load16<T, true>(op[j], of[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < U; ++j) {
    if (!op[j]) continue;
    if (MODE == HYDRA_SCATTER_ADD) {
#pragma unroll
      for (int e = 0; e < E; ++e) of[j][e] = w ? fmaf(wt[j], yf[j][e], of[j][e]) : of[j][e] + yf[j][e];
      store16<T, true>(op[j], of[j]);
    } else {
      store16<T, true>(op[j], yf[j]);
    }
  }
}

template <typename T, int MODE>
__global__ __launch_bounds__(256) void mod_scatter_scalar_kernel(
    T* __restrict__ out, const T* __restrict__ y, const int64_t* __restrict__ idx,
    const float* __restrict__ w, int64_t total, int64_t D, int64_t k, int64_t L,
    int64_t o_bs, int64_t o_ls) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= total) return;
  const int64_t r = t / D, c = t - r * D;
  const int64_t b = r / k;
  const int64_t dst = idx[r];
  if (dst < 0 || dst >= L) return;
  T* op = out + b * o_bs + dst * o_ls + c;
  const float yv = y ? to_f32(y[t]) : 0.f;
  if (MODE == HYDRA_SCATTER_ADD) {
    *op = from_f32<T>(w ? fmaf(w[r], yv, to_f32(*op)) : to_f32(*op) + yv);
  } else {
    *op = from_f32<T>(yv);
  }
}

// Scatter-add that allows repeated indices (torch.scatter_add_ semantics on
// the CPU): thread = (batch row, column); it walks j = 0..k-1 in order and
// updates out[b, idx[b,j], c] += y[b,j,c], rounding after every add, so
// repeats accumulate in index order, deterministically.  Not a hot path (the
// routing wrappers use the distinct-index kernel above).
template <typename T>
__global__ __launch_bounds__(256) void mod_scatter_seq_kernel(
    T* __restrict__ out, const T* __restrict__ y, const int64_t* __restrict__ idx,
    int64_t B, int64_t D, int64_t k, int64_t L, int64_t o_bs, int64_t o_ls) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= B * D) return;
  const int64_t b = t / D, c = t - b * D;
  const int64_t* ir = idx + b * k;
  const T* yr = y + b * k * D + c;
  T* ob = out + b * o_bs + c;
  for (int64_t j = 0; j < k; ++j) {
    const int64_t dst = ir[j];
    if (dst < 0 || dst >= L) continue;
    T* op = ob + dst * o_ls;
    *op = from_f32<T>(to_f32(*op) + to_f32(yr[j * D]));
  }
}

}  // namespace hydra

using namespace hydra;

static int max_lds_per_block() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 65536;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
    return 65536;
  return v;
}

extern "C" int hydra_mod_topk(const void* scores, int64_t B, int64_t L, int64_t s_rs,
                              int64_t k, int64_t* idx_desc, int64_t* idx_sorted,
                              void* mask, int score_dtype, int mask_dtype,
                              void* stream) {
  HYDRA_REQUIRE(B >= 0, "mod_topk: negative batch");
  HYDRA_REQUIRE(L >= 1 && L < (int64_t(1) << 31), "mod_topk: need 1 <= L < 2^31");
  HYDRA_REQUIRE(k >= 1 && k <= L, "mod_topk: need 1 <= k <= L");
  HYDRA_REQUIRE(s_rs >= L, "mod_topk: row stride smaller than L");
  HYDRA_REQUIRE(score_dtype == HYDRA_F32 || score_dtype == HYDRA_BF16 || score_dtype == HYDRA_F16,
                "mod_topk: unknown score dtype code");
  HYDRA_REQUIRE(mask_dtype == HYDRA_F32 || mask_dtype == HYDRA_BF16 || mask_dtype == HYDRA_F16,
                "mod_topk: unknown mask dtype code");
  HYDRA_REQUIRE(B <= 65535, "mod_topk: B must be <= 65535");
  if (B == 0) return HYDRA_OK;
  HYDRA_REQUIRE(scores != nullptr, "mod_topk: null scores");
  // rows beyond the bucket kernel: the device-wide radix sort (the
  // bitonic kernel stays reachable up to kLdsMaxL as a test switch)
  const bool force_bitonic = getenv("HYDRA_TOPK_BITONIC") != nullptr;
  if (L > kLdsMaxL || (L > kBucketMaxL && !force_bitonic))
    return mod_topk_large(scores, B, L, s_rs, k, idx_desc, idx_sorted, mask, score_dtype, mask_dtype,
                          static_cast<hipStream_t>(stream));
  int ept = 1;
  while (ept * kTopkThreads < L) ept <<= 1;
  const int P = ept * kTopkThreads;
  // The bucket kernel's 16K-bin histogram needs ~90-146 KiB of LDS; on a
  // device with less per workgroup the row takes the bitonic kernel, and a
  // row that fits neither takes the device-wide sort.
  const size_t lds_bucket = sizeof(uint64_t) * (P + kKeyPad) + sizeof(uint32_t) * kBinWords +
                            2 * sizeof(uint32_t) * (P / 32);
  const size_t lds_bitonic = sizeof(uint64_t) * P + sizeof(uint32_t) * ((L + 31) / 32);
  const size_t lds_cap = static_cast<size_t>(max_lds_per_block());
  const bool bucket = L <= kBucketMaxL && !force_bitonic && lds_bucket + 1024 <= lds_cap;
  const size_t lds = bucket ? lds_bucket : lds_bitonic;
  const int R = static_cast<int>((L + kTopkThreads - 1) / kTopkThreads);  // bucket kernel: parts per row
  if (lds + 1024 > lds_cap)
    return mod_topk_large(scores, B, L, s_rs, k, idx_desc, idx_sorted, mask, score_dtype, mask_dtype,
                          static_cast<hipStream_t>(stream));
  auto st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(B));
  auto go = [&](auto s_tag, auto e_tag) {
    using ST = decltype(s_tag);
    constexpr int E = decltype(e_tag)::value;
    if (bucket) {
      auto kern = mod_topk_bucket_kernel<ST, (E < 8 ? E : 8)>;
      if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(lds)) != hipSuccess)
        return false;
      kern<<<dim3(static_cast<unsigned>(B * R)), kTopkThreads, lds, st>>>(
          static_cast<const ST*>(scores), (int)L, s_rs, (int)k, R, idx_desc, idx_sorted, mask, mask_dtype);
      return true;
    }
    auto kern = mod_topk_kernel<ST, E>;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) != hipSuccess)
      return false;
    kern<<<grid, kTopkThreads, lds, st>>>(static_cast<const ST*>(scores), (int)L, s_rs, (int)k,
                                          idx_desc, idx_sorted, mask, mask_dtype);
    return true;
  };
  auto by_ept = [&](auto s_tag) -> bool {
    switch (ept) {
      case 1: return go(s_tag, std::integral_constant<int, 1>());
      case 2: return go(s_tag, std::integral_constant<int, 2>());
      case 4: return go(s_tag, std::integral_constant<int, 4>());
      case 8: return go(s_tag, std::integral_constant<int, 8>());
      default: return go(s_tag, std::integral_constant<int, 16>());
    }
  };
  bool set = false;
  switch (score_dtype) {
    case HYDRA_F32: set = by_ept(float()); break;
    case HYDRA_BF16: set = by_ept(bf16()); break;
    case HYDRA_F16: set = by_ept(f16()); break;
    default:
      return fail(HYDRA_ERR_ARG, "mod_topk: unknown score dtype code");
  }
  if (!set) return fail(HYDRA_ERR_LAUNCH, "mod_topk: cannot set the kernel's LDS size");
  return check_launch("mod_topk_kernel");
}

template <typename T>
static int launch_gather(const void* x, const int64_t* idx, void* xs, int64_t B,
                         int64_t L, int64_t k, int64_t D, int64_t x_bs, int64_t x_ls,
                         hipStream_t st) {
  constexpr int E = Vec<T>::N;
  const int64_t cpr = D / E;
  const int64_t total_vec = B * k * cpr;
  const bool vec_ok = D % E == 0 && x_bs % E == 0 && x_ls % E == 0 && aligned16(x) &&
                      aligned16(xs) && total_vec < (int64_t(1) << 31) && B * k < (int64_t(1) << 31);
  if (vec_ok) {
    constexpr int U = 1;
    const dim3 grid(static_cast<unsigned>((total_vec + 256 * U - 1) / (256 * U)));
    mod_gather_kernel<T, U><<<grid, 256, 0, st>>>(static_cast<const T*>(x), idx,
                                                static_cast<T*>(xs), (uint32_t)total_vec,
                                                (uint32_t)cpr, (uint32_t)k, L, x_bs, x_ls);
    return check_launch("mod_gather_kernel");
  }
  const int64_t total = B * k * D;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  mod_gather_scalar_kernel<T><<<grid, 256, 0, st>>>(static_cast<const T*>(x), idx,
                                                     static_cast<T*>(xs), total, D, k, L,
                                                     x_bs, x_ls);
  return check_launch("mod_gather_scalar_kernel");
}

extern "C" int hydra_mod_gather(const void* x, const int64_t* idx, void* xs, int64_t B,
                                int64_t L, int64_t k, int64_t D, int64_t x_bs,
                                int64_t x_ls, int dtype, void* stream) {
  HYDRA_REQUIRE(B >= 0 && L >= 0 && k >= 0 && D >= 0, "mod_gather: negative size");
  if (B * k * D == 0) return HYDRA_OK;
  HYDRA_REQUIRE(x && idx && xs, "mod_gather: null pointer");
  HYDRA_REQUIRE(x_ls >= D, "mod_gather: row stride smaller than D");
  HYDRA_REQUIRE((B * k * D + 255) / 256 < (int64_t(1) << 31), "mod_gather: too large");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    return launch_gather<T>(x, idx, xs, B, L, k, D, x_bs, x_ls, st);
  });
}

template <typename T>
static int launch_scatter(void* out, const void* y, const int64_t* idx, const float* w,
                          int64_t B, int64_t L, int64_t k, int64_t D, int64_t o_bs,
                          int64_t o_ls, int mode, hipStream_t st) {
  constexpr int E = Vec<T>::N;
  const int64_t cpr = D / E;
  const int64_t total_vec = B * k * cpr;
  auto O = static_cast<T*>(out);
  auto Y = static_cast<const T*>(y);
  if (mode == HYDRA_SCATTER_ADD_SEQ) {
    const dim3 grid(static_cast<unsigned>((B * D + 255) / 256));
    mod_scatter_seq_kernel<T><<<grid, 256, 0, st>>>(O, Y, idx, B, D, k, L, o_bs, o_ls);
    return check_launch("mod_scatter_seq_kernel");
  }
  const bool vec_ok = D % E == 0 && o_bs % E == 0 && o_ls % E == 0 && aligned16(out) &&
                      (y == nullptr || aligned16(y)) && total_vec < (int64_t(1) << 31) &&
                      B * k < (int64_t(1) << 31);
  if (vec_ok) {
    constexpr int U = 1;
    const dim3 grid(static_cast<unsigned>((total_vec + 256 * U - 1) / (256 * U)));
    if (mode == HYDRA_SCATTER_ADD)
      mod_scatter_kernel<T, HYDRA_SCATTER_ADD, U><<<grid, 256, 0, st>>>(
          O, Y, idx, w, (uint32_t)total_vec, (uint32_t)cpr, (uint32_t)k, L, o_bs, o_ls);
    else
      mod_scatter_kernel<T, HYDRA_SCATTER_REPLACE, U><<<grid, 256, 0, st>>>(
          O, Y, idx, w, (uint32_t)total_vec, (uint32_t)cpr, (uint32_t)k, L, o_bs, o_ls);
    return check_launch("mod_scatter_kernel");
  }
  const int64_t total = B * k * D;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  if (mode == HYDRA_SCATTER_ADD)
    mod_scatter_scalar_kernel<T, HYDRA_SCATTER_ADD><<<grid, 256, 0, st>>>(
        O, Y, idx, w, total, D, k, L, o_bs, o_ls);
  else
    mod_scatter_scalar_kernel<T, HYDRA_SCATTER_REPLACE><<<grid, 256, 0, st>>>(
        O, Y, idx, w, total, D, k, L, o_bs, o_ls);
  return check_launch("mod_scatter_scalar_kernel");
}

extern "C" int hydra_mod_scatter(void* out, const void* y, const int64_t* idx,
                                 const float* w, int64_t B, int64_t L, int64_t k,
                                 int64_t D, int64_t o_bs, int64_t o_ls, int mode,
                                 int dtype, void* stream) {
  HYDRA_REQUIRE(B >= 0 && L >= 0 && k >= 0 && D >= 0, "mod_scatter: negative size");
  HYDRA_REQUIRE(mode == HYDRA_SCATTER_ADD || mode == HYDRA_SCATTER_REPLACE ||
                    mode == HYDRA_SCATTER_ADD_SEQ,
                "mod_scatter: unknown mode");
  HYDRA_REQUIRE(w == nullptr || mode == HYDRA_SCATTER_ADD,
                "mod_scatter: weights apply to the ADD mode only");
  if (B * k * D == 0) return HYDRA_OK;
  HYDRA_REQUIRE(out && idx, "mod_scatter: null pointer");
  HYDRA_REQUIRE(y != nullptr || mode == HYDRA_SCATTER_REPLACE,
                "mod_scatter: values may be NULL in the REPLACE mode only");
  HYDRA_REQUIRE(mode != HYDRA_SCATTER_ADD_SEQ || B * D < (int64_t(1) << 40),
                "mod_scatter: too large");
  HYDRA_REQUIRE(o_ls >= D, "mod_scatter: row stride smaller than D");
  HYDRA_REQUIRE((B * k * D + 255) / 256 < (int64_t(1) << 31), "mod_scatter: too large");
  auto st = static_cast<hipStream_t>(stream);
  return HYDRA_DISPATCH_DTYPE(dtype, T, [&] {
    return launch_scatter<T>(out, y, idx, w, B, L, k, D, o_bs, o_ls, mode, st);
  });
}
