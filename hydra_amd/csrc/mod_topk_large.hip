// MoD top-k for rows longer than the in-LDS kernels take (L > 16384): the
// same selection and order as the bucket and bitonic kernels in
// mod_route.hip (value-descending, ties to the lower index, NaN largest,
// -0.0 == +0.0; torch.topk at hydra/routing/mixture_of_depths.py:186), with
// the row's keys sorted in global memory.
//
//  1. every element becomes the composite (row << (32 + ib)) | (desc << ib)
//     | index, where desc = ~score_key_asc(score), ib = bits of L - 1 and rb
//     = bits of B - 1, so an ascending sort keeps the rows apart and orders
//     each row stably value-descending; rb + ib <= 32 whenever B * L < 2^31,
//     so the composite fits 64 bits;
//  2. all composites are radix-sorted together over their rb + 32 + ib bits
//     (hipCUB's device-wide radix sort, which spreads over the whole GPU;
//     a sort per row would give each row one workgroup);
//  3. the first k sorted composites of a row give idx_desc, and its k-th is
//     the row's threshold T: element i is selected iff its composite <= T;
//  4. per chunk of kChunk elements of a row, the count of selected elements;
//  5. per chunk, the mask and, after the counts of the row's earlier chunks
//     and a block prefix count inside the chunk, its ascending list entries.
// The workspace (two composite arrays, the chunk counts and the sort's
// scratch) is stream-ordered: hipMallocAsync before the kernels and
// hipFreeAsync after them on the caller's stream.
#include <hipcub/hipcub.hpp>

#include "common.h"
#include "mod_keys.h"

namespace hydra {
namespace {

constexpr int kChunkThreads = 256;
constexpr int kChunkPer = 8;                              // elements per thread
constexpr int64_t kChunk = kChunkThreads * kChunkPer;     // elements per chunk
static_assert(kChunkThreads % 256 == 0, "wave totals are read in int4 groups");

template <typename S>
__device__ __forceinline__ uint64_t composite(const S* __restrict__ scores, int64_t s_rs, int64_t b,
                                              int64_t i, int ib) {
  const uint32_t desc = ~score_key_asc(to_f32(scores[b * s_rs + i]));
  return (static_cast<uint64_t>(b) << (32 + ib)) | (static_cast<uint64_t>(desc) << ib) |
         static_cast<uint64_t>(i);
}

template <typename S>
__global__ __launch_bounds__(256) void topk_large_keys_kernel(
    const S* __restrict__ scores, int64_t s_rs, int64_t L, int64_t B, int ib,
    uint64_t* __restrict__ keys) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (g >= B * L) return;
  const int64_t b = g / L;
  keys[g] = composite(scores, s_rs, b, g - b * L, ib);
}

__global__ __launch_bounds__(256) void topk_large_emit_kernel(
    const uint64_t* __restrict__ sorted, int64_t L, int64_t k, int64_t B, int ib,
    int64_t* __restrict__ idx_desc) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (g >= B * k) return;
  const int64_t b = g / k, j = g - b * k;
  idx_desc[g] = static_cast<int64_t>(sorted[b * L + j] & ((uint64_t(1) << ib) - 1));
}

// Block-wide exclusive prefix of `v` (kChunkThreads threads); *total gets
// the sum.  Uses wave_tot[kChunkThreads / 64] and two barriers.
__device__ __forceinline__ int block_excl_sum(int v, int* wave_tot, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int incl = wave_incl_sum(v);
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  int base = 0, all = 0;
#pragma unroll
  for (int q = 0; q < kChunkThreads / 256; ++q) {
    const int4 t = reinterpret_cast<const int4*>(wave_tot)[q];
    const int tv[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      base += 4 * q + u < wave ? tv[u] : 0;
      all += tv[u];
    }
  }
  __syncthreads();  // wave_tot may be rewritten after return
  *total = all;
  return base + incl - v;
}

// grid (chunks, B): thread t takes elements c*kChunk + kChunkPer*t + [0, kChunkPer)
template <typename S>
__global__ __launch_bounds__(kChunkThreads) void topk_large_count_kernel(
    const S* __restrict__ scores, int64_t s_rs, int64_t L, int ib, const uint64_t* __restrict__ sorted,
    int64_t k, int* __restrict__ counts) {
  __shared__ __attribute__((aligned(16))) int wave_tot[kChunkThreads / 64];
  const int64_t b = blockIdx.y, c = blockIdx.x, nchunks = gridDim.x;
  const uint64_t T = sorted[b * L + k - 1];
  const int64_t i0 = c * kChunk + kChunkPer * static_cast<int64_t>(threadIdx.x);
  int n = 0;
#pragma unroll
  for (int j = 0; j < kChunkPer; ++j)
    n += (i0 + j < L && composite(scores, s_rs, b, i0 + j, ib) <= T) ? 1 : 0;
  int total;
  block_excl_sum(n, wave_tot, &total);
  if (threadIdx.x == 0) counts[b * nchunks + c] = total;
}

template <typename S>
__global__ __launch_bounds__(kChunkThreads) void topk_large_list_kernel(
    const S* __restrict__ scores, int64_t s_rs, int64_t L, int ib, const uint64_t* __restrict__ sorted,
    int64_t k, const int* __restrict__ counts, int64_t* __restrict__ idx_sorted, void* __restrict__ mask,
    int mask_dtype) {
  __shared__ __attribute__((aligned(16))) int wave_tot[kChunkThreads / 64];
  const int64_t b = blockIdx.y, c = blockIdx.x, nchunks = gridDim.x;
  const uint64_t T = sorted[b * L + k - 1];
  const int64_t i0 = c * kChunk + kChunkPer * static_cast<int64_t>(threadIdx.x);
  uint32_t sel = 0u;
#pragma unroll
  for (int j = 0; j < kChunkPer; ++j)
    if (i0 + j < L && composite(scores, s_rs, b, i0 + j, ib) <= T) sel |= 1u << j;
  if (mask) {
    const int64_t mrow = b * L;
#pragma unroll
    for (int j = 0; j < kChunkPer; ++j) {
      if (i0 + j >= L) break;
      const float v = (sel >> j) & 1u ? 1.f : 0.f;
      switch (mask_dtype) {
        case HYDRA_F32: static_cast<float*>(mask)[mrow + i0 + j] = v; break;
        case HYDRA_BF16: static_cast<bf16*>(mask)[mrow + i0 + j] = from_f32<bf16>(v); break;
        default: static_cast<f16*>(mask)[mrow + i0 + j] = from_f32<f16>(v); break;
      }
    }
  }
  if (!idx_sorted) return;
  // selected elements of the row's earlier chunks
  int before = 0;
  for (int64_t q = threadIdx.x; q < c; q += kChunkThreads) before += counts[b * nchunks + q];
  int total;
  block_excl_sum(before, wave_tot, &total);
  const int64_t base = total;
  int64_t pos = base + block_excl_sum(__popc(sel), wave_tot, &total);
  int64_t* orow = idx_sorted + b * k;
  while (sel) {
    const int j = __ffs(sel) - 1;
    sel &= sel - 1;
    if (pos < k) orow[pos] = i0 + j;
    ++pos;
  }
}

size_t align_up(size_t v) { return (v + 255) & ~size_t(255); }

}  // namespace

int mod_topk_large(const void* scores, int64_t B, int64_t L, int64_t s_rs, int64_t k,
                   int64_t* idx_desc, int64_t* idx_sorted, void* mask, int score_dtype,
                   int mask_dtype, hipStream_t st) {
  // hipCUB's item count is int
  if (B * L >= (int64_t(1) << 31))
    return fail(HYDRA_ERR_UNSUPPORTED, "mod_topk: B * L must be < 2^31 for rows longer than 8192");
  int ib = 0, rb = 0;
  while ((int64_t(1) << ib) < L) ++ib;
  while ((int64_t(1) << rb) < B) ++rb;
  const int end_bit = rb + 32 + ib;  // <= 64 since B * L < 2^31
  const int n = static_cast<int>(B * L);
  const int64_t nchunks = (L + kChunk - 1) / kChunk;
  size_t temp = 0;
  if (hipcub::DeviceRadixSort::SortKeys(nullptr, temp, static_cast<const uint64_t*>(nullptr),
                                        static_cast<uint64_t*>(nullptr), n, 0, end_bit, st) != hipSuccess)
    return fail(HYDRA_ERR_LAUNCH, "mod_topk: radix sort size query failed");
  const size_t keys_b = align_up(sizeof(uint64_t) * static_cast<size_t>(B * L));
  const size_t cnt_b = align_up(sizeof(int) * static_cast<size_t>(B * nchunks));
  const size_t total = 2 * keys_b + cnt_b + align_up(temp);
  void* ws = nullptr;
  if (hipMallocAsync(&ws, total, st) != hipSuccess) {
    (void)hipGetLastError();
    return fail(HYDRA_ERR_LAUNCH, "mod_topk: cannot allocate the long-row workspace");
  }
  auto* base = static_cast<unsigned char*>(ws);
  auto* keys_in = reinterpret_cast<uint64_t*>(base);
  auto* keys_out = reinterpret_cast<uint64_t*>(base + keys_b);
  auto* counts = reinterpret_cast<int*>(base + 2 * keys_b);
  void* tmp = base + 2 * keys_b + cnt_b;

  const dim3 g1(static_cast<unsigned>((B * L + 255) / 256));
  const dim3 gc(static_cast<unsigned>(nchunks), static_cast<unsigned>(B));
  auto run = [&](auto s_tag) -> int {
    using S = decltype(s_tag);
    const S* sc = static_cast<const S*>(scores);
    topk_large_keys_kernel<S><<<g1, 256, 0, st>>>(sc, s_rs, L, B, ib, keys_in);
    int rc = check_launch("topk_large_keys_kernel");
    if (rc != HYDRA_OK) return rc;
    if (hipcub::DeviceRadixSort::SortKeys(tmp, temp, keys_in, keys_out, n, 0, end_bit, st) != hipSuccess)
      return fail(HYDRA_ERR_LAUNCH, "mod_topk: radix sort launch failed");
    if (idx_desc) {
      topk_large_emit_kernel<<<dim3(static_cast<unsigned>((B * k + 255) / 256)), 256, 0, st>>>(
          keys_out, L, k, B, ib, idx_desc);
      if ((rc = check_launch("topk_large_emit_kernel")) != HYDRA_OK) return rc;
    }
    if (idx_sorted) {
      topk_large_count_kernel<S><<<gc, kChunkThreads, 0, st>>>(sc, s_rs, L, ib, keys_out, k, counts);
      if ((rc = check_launch("topk_large_count_kernel")) != HYDRA_OK) return rc;
    }
    if (idx_sorted || mask) {
      topk_large_list_kernel<S><<<gc, kChunkThreads, 0, st>>>(sc, s_rs, L, ib, keys_out, k, counts, idx_sorted,
                                                              mask, mask_dtype);
      if ((rc = check_launch("topk_large_list_kernel")) != HYDRA_OK) return rc;
    }
    return HYDRA_OK;
  };
  int rc;
  switch (score_dtype) {
    case HYDRA_F32: rc = run(float()); break;
    case HYDRA_BF16: rc = run(bf16()); break;
    default: rc = run(f16()); break;
  }
  if (hipFreeAsync(ws, st) != hipSuccess && rc == HYDRA_OK)
    rc = fail(HYDRA_ERR_LAUNCH, "mod_topk: cannot release the long-row workspace");
  return rc;
}

}  // namespace hydra
