// Shared device/host helpers of the gfx950 kernels: element types, 16-byte
// vector I/O, wave64 reductions and the error plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>
#include <type_traits>

#include "../../include/hydra_amd.h"

namespace hydra {

// ---- element types ------------------------------------------------------
// bf16 and fp16 are carried as raw 16-bit patterns; every kernel converts to
// fp32, computes in fp32 and rounds once (round-to-nearest-even) on store.
struct bf16 { uint16_t bits; };
struct f16 { uint16_t bits; };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) {
  return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}
__device__ __forceinline__ float to_f32(f16 v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, v.bits));
}

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) {
  // gfx950 converts in hardware (v_cvt_pk_bf16_f32): round to nearest even,
  // NaN stays NaN.
  bf16 r;
  r.bits = __builtin_bit_cast(uint16_t, static_cast<__bf16>(v));
  return r;
}
template <> __device__ __forceinline__ f16 from_f32<f16>(float v) {
  f16 r;
  r.bits = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
  return r;
}

// Two values rounded to a 16-bit type, packed low | high << 16 (one
// v_cvt_pk_bf16_f32 for bf16).
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (sizeof(T) == 2 && std::is_same<T, bf16>::value) {
    typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
    const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    return static_cast<uint32_t>(from_f32<T>(lo).bits) |
           (static_cast<uint32_t>(from_f32<T>(hi).bits) << 16);
  }
}

// Elements of T in one 16-byte vector.
template <typename T> struct Vec { static constexpr int N = 16 / sizeof(T); };

// 16-byte load / store of N elements of T, converted to / from fp32.  NT
// marks the access non-temporal (streamed once: no allocation in L2/MALL),
// which gains ~7% of HBM bandwidth on pure streaming kernels on gfx950.
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_nt;

template <bool NT>
__device__ __forceinline__ uint4 ld16raw(const void* p) {
  if constexpr (NT) {
    const u32x4_nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const uint4*>(p);
  }
}

template <bool NT>
__device__ __forceinline__ void st16raw(void* p, uint4 v) {
  if constexpr (NT) {
    const u32x4_nt w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4_nt*>(p));
  } else {
    *reinterpret_cast<uint4*>(p) = v;
  }
}

template <typename T>
__device__ __forceinline__ void unpack16(const uint4 raw, float* out) {
  if constexpr (sizeof(T) == 4) {
    out[0] = __uint_as_float(raw.x); out[1] = __uint_as_float(raw.y);
    out[2] = __uint_as_float(raw.z); out[3] = __uint_as_float(raw.w);
  } else {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      T lo, hi;
      lo.bits = static_cast<uint16_t>(w[i] & 0xffffu);
      hi.bits = static_cast<uint16_t>(w[i] >> 16);
      out[2 * i] = to_f32(lo);
      out[2 * i + 1] = to_f32(hi);
    }
  }
}

template <typename T>
__device__ __forceinline__ uint4 pack16(const float* in) {
  uint4 raw;
  if constexpr (sizeof(T) == 4) {
    raw.x = __float_as_uint(in[0]); raw.y = __float_as_uint(in[1]);
    raw.z = __float_as_uint(in[2]); raw.w = __float_as_uint(in[3]);
  } else {
    raw.x = pack2<T>(in[0], in[1]); raw.y = pack2<T>(in[2], in[3]);
    raw.z = pack2<T>(in[4], in[5]); raw.w = pack2<T>(in[6], in[7]);
  }
  return raw;
}

template <typename T, bool NT = false>
__device__ __forceinline__ void load16(const T* p, float* out) {
  unpack16<T>(ld16raw<NT>(p), out);
}

template <typename T, bool NT = false>
__device__ __forceinline__ void store16(T* p, const float* in) {
  st16raw<NT>(p, pack16<T>(in));
}

// ---- wave64 reductions ---------------------------------------------------
template <int WIDTH = 64>
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, WIDTH);
  return v;
}
template <int WIDTH = 64>
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, WIDTH));
  return v;
}

// x combined with its copy in the other half of the wave (lane l ^ 32),
// through v_permlane32_swap: a = (x[0..31], x[0..31]), b = (x[32..63],
// x[32..63]), so max(a, b) and a + b hold the pair's max and sum in every
// lane (both halves get the same bits: + is commutative).
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---- host-side error plumbing -------------------------------------------
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);
bool aligned16(const void* p);
int dtype_size(int dtype);
// Compute units of the current device (cached per device).
int device_cus();
// Workgroups of `kernel` (launched with `threads`) resident on one CU.
int blocks_per_cu(const void* kernel, int threads);

}  // namespace hydra

#define HYDRA_REQUIRE(cond, msg)                                 \
  do {                                                           \
    if (!(cond)) return ::hydra::fail(HYDRA_ERR_ARG, (msg));     \
  } while (0)

// Dispatch a templated launcher over the three element types.
#define HYDRA_DISPATCH_DTYPE(dtype, T, ...)                                   \
  [&]() -> int {                                                             \
    switch (dtype) {                                                         \
      case HYDRA_F32: { using T = float; return __VA_ARGS__(); }            \
      case HYDRA_BF16: { using T = ::hydra::bf16; return __VA_ARGS__(); }   \
      case HYDRA_F16: { using T = ::hydra::f16; return __VA_ARGS__(); }     \
      default: return ::hydra::fail(HYDRA_ERR_ARG, "unknown dtype code");    \
    }                                                                        \
  }()
