// Projection with a short reduction on gfx950: y = x W^T (F.linear without
// bias) for bf16 when K <= 256 -- the CCGQA output projection o_proj
// (hydra/attention/backends/ccgqa/attention.py:329-331), K = latent dim.
//
// Weight-stationary: each wave holds a 32-column slice of W (32 x K bf16,
// 64 VGPRs at K = 256) in registers, so W is read once per workgroup; the
// workgroup's 8 waves cover 256 output columns of 256 rows of x, staged in
// LDS at once (loads of x issued before those of W, one barrier), then
// multiplied in 32-row blocks with no barrier between them.  The grid is
// one-dimensional and XCD-aware: workgroup ids congruent mod 8 run on one
// XCD, and the column groups of a row group get such ids, so the x rows one
// of them stages are L2 hits for the others.  Against 64-column slices of
// 128 rows (half the x reads, twice the weight bytes per CU): 14.5 us
// against 15.7 at [16384, 256] x [1024, 256]; without the XCD mapping the
// 256-row tiles take 17.4.
// Per block a wave runs K/16 k-steps x 2 MFMAs (v_mfma_f32_32x32x16_bf16)
// with its weight fragments as the A operand and the staged rows as the B
// operand, so the accumulator holds y^T: lane (m, half) owns row m and
// columns 8 g + 4 half + 0..3; a v_permlane32_swap between the halves gives
// each lane 8 consecutive columns, stored as one 16-byte write.  fp32
// accumulation, one rounding to bf16 (as the library GEMM).
#include "common.h"

#include <type_traits>

namespace hydra {
namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_l;
typedef __attribute__((ext_vector_type(16))) float f32x16_l;

constexpr int kLinWaves = 8;   // waves per workgroup
constexpr int kLinNCW = 32;    // output columns per wave
constexpr int kLinRB = 32;     // rows per block step
constexpr int kLinRows = 256;  // rows per workgroup
constexpr int kLinCols = kLinWaves * kLinNCW;  // columns per workgroup

__device__ __forceinline__ bf16x8_l as_b8(uint4 v) { return __builtin_bit_cast(bf16x8_l, v); }

template <int K, bool TILED>
__global__ __launch_bounds__(64 * kLinWaves) void linear_ws_kernel(
    const bf16* __restrict__ x, int64_t x_rs, const bf16* __restrict__ w, int64_t w_rs,
    bf16* __restrict__ y, int64_t y_rs, int M, int N) {
  constexpr int KS = K / 16;             // k-steps
  constexpr int NB = kLinNCW / 32;       // 32-column blocks per wave
  constexpr int XP = K + 8;              // LDS row pitch (elements): rows 16 bytes apart in bank
  constexpr int XC = K / 8;              // 16-byte chunks per row
  constexpr int NT = 64 * kLinWaves;
  constexpr int CPT = (kLinRows * XC + NT - 1) / NT;  // x chunks per thread
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];  // kLinRows rows of x
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, hf = lane >> 5;
  // workgroup id -> (column group, row group): ids xcd + 8 * sl share an XCD;
  // sl runs over the column groups of row group (sl / ncg) * 8 + xcd
  const int ncg = (N + kLinCols - 1) / kLinCols;
  const int id = blockIdx.x, xcd = id & 7, sl = id >> 3;
  const int cg = sl % ncg, rg = (sl / ncg) * 8 + xcd;
  const int r0 = rg * kLinRows;
  if (r0 >= M) return;  // the row groups are rounded up to a multiple of 8
  const int c0 = cg * kLinCols + wave * kLinNCW;  // the wave's first column
  const bool wact = c0 < N;  // N % 32 == 0: a wave's columns are all in range or none
  const int r1 = min(M, r0 + kLinRows);

  // The workgroup's rows of x first (rows at or past r1 read as 0; their
  // outputs are not stored), then the weights, so the x rows land first.
  uint4 xv[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int i = tid + j * NT;
    const int row = i / XC, ch = i - row * XC;
    xv[j] = make_uint4(0, 0, 0, 0);
    if (i < kLinRows * XC && r0 + row < r1)
      xv[j] = *reinterpret_cast<const uint4*>(x + static_cast<int64_t>(r0 + row) * x_rs + 8 * ch);
  }
  // The wave's weight fragments: wf[nb][s] = W[c0 + 32 nb + n][16 s + 8 hf .. +7],
  // in the order the MFMAs use them.  TILED: W in MFMA-fragment order
  // [N/32][K/16][64 lanes][8], one contiguous 1 KB block per fragment (one
  // coalesced load); row-major W makes each load touch 32 rows.
  uint4 wf[NB][KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const bf16* src = TILED ? w + ((static_cast<int64_t>(c0 / 32 + nb) * KS + s) * 64 + lane) * 8
                              : w + static_cast<int64_t>(c0 + 32 * nb + n) * w_rs + 16 * s + 8 * hf;
      wf[nb][s] = wact ? *reinterpret_cast<const uint4*>(src) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    const int i = tid + j * NT;
    const int row = i / XC, ch = i - row * XC;
    if (i < kLinRows * XC) *reinterpret_cast<uint4*>(&xs[row * XP + 8 * ch]) = xv[j];
  }
  __syncthreads();
  if (!wact) return;
  // 32-row blocks, no barrier between them: a block's stores drain behind
  // the next block's MFMAs.
  for (int rb = r0; rb < r1; rb += kLinRB) {
    f32x16_l acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nb][r] = 0.f;
    const uint16_t* xb = xs + (rb - r0 + n) * XP + 8 * hf;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const bf16x8_l b = as_b8(*reinterpret_cast<const uint4*>(xb + 16 * s));
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_b8(wf[nb][s]), b, acc[nb], 0, 0, 0);
    }
    // acc[nb][r] = y[rb + n][c0 + 32 nb + 8 (r / 4) + 4 hf + r % 4]; groups
    // 2p and 2p + 1 swap halves, so lane hf holds columns 8 (2p + hf) .. +7.
    const int m = rb + n;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const f32x16_l& a = acc[nb];
        const uint32_t r0x = pack2<bf16>(a[8 * p + 0], a[8 * p + 1]);
        const uint32_t r0y = pack2<bf16>(a[8 * p + 2], a[8 * p + 3]);
        const uint32_t r1x = pack2<bf16>(a[8 * p + 4], a[8 * p + 5]);
        const uint32_t r1y = pack2<bf16>(a[8 * p + 6], a[8 * p + 7]);
        const auto sx = __builtin_amdgcn_permlane32_swap(r0x, r1x, false, false);
        const auto sy = __builtin_amdgcn_permlane32_swap(r0y, r1y, false, false);
        const int col = c0 + 32 * nb + 8 * (2 * p + hf);
        if (m < r1)
          *reinterpret_cast<uint4*>(y + static_cast<int64_t>(m) * y_rs + col) =
              make_uint4(sx[0], sy[0], sx[1], sy[1]);
      }
  }
}

}  // namespace
}  // namespace hydra

using namespace hydra;

extern "C" int hydra_linear_fwd(const void* x, int64_t x_rs, const void* w, int64_t w_rs, void* y,
                                int64_t y_rs, int64_t M, int64_t N, int64_t K, int flags, int dtype,
                                void* stream) {
  HYDRA_REQUIRE(M >= 0 && N >= 1 && K >= 1, "linear: bad size");
  HYDRA_REQUIRE((flags & ~HYDRA_LINEAR_W_TILED) == 0, "linear: unknown flag bits");
  const bool tiled = flags & HYDRA_LINEAR_W_TILED;
  HYDRA_REQUIRE(x_rs >= K && (tiled || w_rs >= K) && y_rs >= N, "linear: row stride smaller than the row");
  if (dtype != HYDRA_BF16 || !(K == 64 || K == 128 || K == 256) || N % 64 != 0)
    return fail(HYDRA_ERR_UNSUPPORTED, "linear: takes bf16 with K in {64, 128, 256} and N % 64 == 0");
  if (M == 0) return HYDRA_OK;
  HYDRA_REQUIRE(x && w && y, "linear: null pointer");
  if (x_rs % 8 != 0 || (!tiled && w_rs % 8 != 0) || y_rs % 8 != 0 || !aligned16(x) || !aligned16(w) ||
      !aligned16(y))
    return fail(HYDRA_ERR_UNSUPPORTED, "linear: needs 16-byte aligned rows");
  HYDRA_REQUIRE(M < (int64_t(1) << 31) && N < (int64_t(1) << 31), "linear: too large");
  auto st = static_cast<hipStream_t>(stream);
  const int64_t ncg = (N + kLinCols - 1) / kLinCols;
  const int64_t nrg = ((M + kLinRows - 1) / kLinRows + 7) / 8 * 8;
  HYDRA_REQUIRE(ncg * nrg < (int64_t(1) << 31), "linear: too large");
  const dim3 grid(static_cast<unsigned>(ncg * nrg));
  auto X = static_cast<const bf16*>(x);
  auto W = static_cast<const bf16*>(w);
  auto Y = static_cast<bf16*>(y);
  auto go = [&](auto k_tag) {
    constexpr int KK = decltype(k_tag)::value;
    const size_t lds = static_cast<size_t>(kLinRows) * (KK + 8) * 2;
    auto kern = tiled ? linear_ws_kernel<KK, true> : linear_ws_kernel<KK, false>;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)) != hipSuccess)
      return fail(HYDRA_ERR_LAUNCH, "linear: cannot set the kernel's LDS size");
    kern<<<grid, 64 * kLinWaves, lds, st>>>(X, x_rs, W, w_rs, Y, y_rs, (int)M, (int)N);
    return check_launch("linear_ws_kernel");
  };
  if (K == 64) return go(std::integral_constant<int, 64>());
  if (K == 128) return go(std::integral_constant<int, 128>());
  return go(std::integral_constant<int, 256>());
}
