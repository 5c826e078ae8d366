// Error plumbing and version query of the C ABI.
#include "common.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>

namespace hydra {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(HYDRA_ERR_LAUNCH,
                std::string(what) + ": " + hipGetErrorString(e));
  }
  return HYDRA_OK;
}

bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

int dtype_size(int dtype) {
  switch (dtype) {
    case HYDRA_F32: return 4;
    case HYDRA_BF16: return 2;
    case HYDRA_F16: return 2;
    default: return 0;
  }
}

int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// From the kernel's register and LDS footprint: a SIMD holds 512 VGPRs per
// lane (allocated in granules of 8) and at most 8 waves, a CU 4 SIMDs and
// 160 KiB of LDS.  (The runtime's occupancy query over-counted for these
// kernels.)
int blocks_per_cu(const void* kernel, int threads) {
  static std::mutex mu;
  static std::map<const void*, int> cache;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(kernel);
  if (it != cache.end()) return it->second;
  hipFuncAttributes a{};
  int nb = 1;
  if (hipFuncGetAttributes(&a, kernel) == hipSuccess) {
    const int regs = std::max(8, (a.numRegs + 7) / 8 * 8);
    const int waves_per_simd = std::min(8, 512 / regs);
    const int waves_per_wg = (threads + 63) / 64;
    const int by_regs = waves_per_simd * 4 / waves_per_wg;
    const size_t lds = a.sharedSizeBytes;
    const int by_lds = lds > 0 ? static_cast<int>((160 * 1024) / lds) : by_regs;
    nb = std::max(1, std::min(by_regs, by_lds));
  }
  if (const char* e = getenv("HYDRA_OCC_DEBUG"))
    if (atoi(e)) fprintf(stderr, "hydra_amd: %d resident workgroups per CU (regs %d, lds %zu)\n", nb, a.numRegs, a.sharedSizeBytes);
  cache[kernel] = nb;
  return nb;
}


}  // namespace hydra

extern "C" const char* hydra_last_error(void) {
  return hydra::g_last_error.c_str();
}

extern "C" int hydra_abi_version(void) { return 111; }

// ---- same-device HBM copy (measurement aid) ---------------------------------
// One 16-byte chunk per thread, non-temporal load and store, 256-thread
// blocks: the fastest plain copy form measured for tens of MB on gfx950
// (non-temporal 10.0 us against 11.4 us cached for 25 MB each way).
namespace hydra {
namespace {
__global__ __launch_bounds__(256) void stream_copy_kernel(const uint4* __restrict__ src,
                                                          uint4* __restrict__ dst, int64_t n) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t < n) st16raw<true>(dst + t, ld16raw<true>(src + t));
}
}  // namespace
}  // namespace hydra

extern "C" int hydra_stream_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  using namespace hydra;
  HYDRA_REQUIRE(bytes >= 0 && bytes % 16 == 0, "stream_copy: bytes must be a non-negative multiple of 16");
  if (bytes == 0) return HYDRA_OK;
  HYDRA_REQUIRE(src && dst, "stream_copy: null pointer");
  HYDRA_REQUIRE(aligned16(src) && aligned16(dst), "stream_copy: pointers must be 16-byte aligned");
  const int64_t n = bytes / 16;
  HYDRA_REQUIRE((n + 255) / 256 < (int64_t(1) << 31), "stream_copy: too large");
  stream_copy_kernel<<<dim3(static_cast<unsigned>((n + 255) / 256)), 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(src), static_cast<uint4*>(dst), n);
  return check_launch("stream_copy_kernel");
}

// ---- shader clock under matrix-core load (measurement aid) -----------------
// Each workgroup of 8 waves (two per SIMD) issues v_mfma_f32_32x32x16_bf16
// into four independent accumulators and v_exp_f32 on 16 independent chains
// per iteration, the attention tile's two instruction kinds, and stamps the
// shader clock (s_memtime) and the constant-rate wall clock
// (s_memrealtime) before and after, between workgroup barriers.
namespace hydra {
namespace {
typedef __attribute__((ext_vector_type(8))) __bf16 probe_bf16x8_t;
typedef __attribute__((ext_vector_type(16))) float probe_f32x16_t;

__global__ __launch_bounds__(512) void clock_probe_kernel(unsigned long long* __restrict__ stamps, int iters) {
  const int lane = threadIdx.x & 63;
  const uint4 raw = make_uint4(0x3f803f80u ^ lane, 0x3f803f80u, 0x3c003c00u, 0x3f003f00u);
  const probe_bf16x8_t a = __builtin_bit_cast(probe_bf16x8_t, raw);
  probe_f32x16_t acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
  float e[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) e[j] = 0.01f * (lane + j);
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, a, acc[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 16; ++j) e[j] = __builtin_amdgcn_exp2f(-0.5f * e[j]);
  }
  __syncthreads();
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  float sink = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) sink += acc[j][lane & 15];
#pragma unroll
  for (int j = 0; j < 16; ++j) sink += e[j];
  if (threadIdx.x == 0) {
    unsigned long long* o = stamps + 5 * static_cast<int64_t>(blockIdx.x);
    o[0] = t0;
    o[1] = t1;
    o[2] = r0;
    o[3] = r1;
    o[4] = static_cast<unsigned long long>(__float_as_uint(sink));
  }
}
}  // namespace
}  // namespace hydra

extern "C" int hydra_clock_probe(void* stamps, int nwg, int iters, int64_t* wall_khz, void* stream) {
  using namespace hydra;
  HYDRA_REQUIRE(stamps != nullptr && wall_khz != nullptr, "clock_probe: null pointer");
  HYDRA_REQUIRE(nwg >= 1 && nwg <= 65535, "clock_probe: need 1 <= nwg <= 65535");
  HYDRA_REQUIRE(iters >= 1, "clock_probe: need iters >= 1");
  HYDRA_REQUIRE(reinterpret_cast<uintptr_t>(stamps) % 8 == 0, "clock_probe: stamps must be 8-byte aligned");
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz <= 0)
    return fail(HYDRA_ERR_LAUNCH, "clock_probe: no wall-clock rate for this device");
  *wall_khz = khz;
  clock_probe_kernel<<<dim3(static_cast<unsigned>(nwg)), 512, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<unsigned long long*>(stamps), iters);
  return check_launch("clock_probe_kernel");
}
