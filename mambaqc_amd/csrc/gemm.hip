// Hand-written MFMA GEMM for the block's B/C projections (bf16 or fp16):
//   C[M, N] = X[M, K] . W[N, K]^T,  fp32 accumulation, output in the operands' type,
// the nn.Linear layout of mambaqc/layers/quaternion_linear.py:145-161
// (F.linear(x, W) for the real -> quaternion maps B_proj and C_proj,
// models/quaternion_mamba2_block.py:186-191).
//
// This is the first stage of fusing the projections with the SSM walk: a
// GEMM whose tile loop this library owns. It is exported and tested, and
// measured against hipBLASLt on the same shapes; the block keeps hipBLASLt,
// which is faster at the config-3 shape (M 8192, N 393216, K 1536).
//
// Tiling (gfx950): the 256 x 256 MFMA main loop of mfma_tile.hpp (8 waves, two 64 KB
// LDS stages filled by global->LDS DMA, 16 x 16 x 32 bf16 or fp16 MFMAs), plus:
//   - Tiles in launch order with the M tile fastest: the 256 tiles in flight cover all of X
//     (in the Infinity Cache) and a few W tiles, each of which is read from HBM about once.
//   - Epilogue through LDS: the tile is written to LDS in the MFMA layout (rows of 512 bytes,
//     16-byte chunks XORed with row & 31) and read back as whole rows, so every global
//     store writes 16 bytes per lane along a row (nontemporal: C is not read back here).
// Rows of X past M are clamped onto row M - 1 for the loads and never stored, so M is
// free; N must be a multiple of 256 and K of 64.
#include <atomic>

#include "mfma_tile.hpp"

namespace mqc {
namespace {

using namespace mfma;

constexpr int kGT = kT;
constexpr int kGBK = kBK;
constexpr int kGThreads = kThreads;
constexpr int kLdsBytes = kStagesBytes;  // two stages = 128 KB (also the epilogue tile)

// One 256 x 256 tile. T: the 16-bit storage type (bf16_t or f16_t). FULL_M: all 256
// rows of the tile exist (every row tile but a ragged last one, whose rows past M read
// row M - 1).
template <typename T, bool FULL_M>
__device__ inline void gemm_tile(const uint16_t* __restrict__ X, const uint16_t* __restrict__ W,
                                 uint16_t* __restrict__ C, int M, int N, int K, int m0, int n0,
                                 char* lds) {
  using E = typename std::conditional<std::is_same<T, bf16_t>::value, __bf16, _Float16>::type;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave >> 2;
  const int wm = wave & 3;
  const int rl = lane & 15;
  const int q = lane >> 4;
  floatx4 acc[kWB][kXB];
#pragma unroll
  for (int a = 0; a < kWB; ++a)
#pragma unroll
    for (int b = 0; b < kXB; ++b) acc[a][b] = (floatx4){};
  auto wrow = [&](int g, int k0, int i, uint32_t& voff, const DmaLane& dl) -> const void* {
    voff = (uint32_t)(dl.lrow * K * 2) + dl.cb(i);
    return W + ((int64_t)(n0 + g) * K + k0);
  };
  auto xrow = [&](int g, int k0, int i, uint32_t& voff, const DmaLane& dl) -> const void* {
    if constexpr (FULL_M) {
      voff = (uint32_t)(dl.lrow * K * 2) + dl.cb(i);
      return X + ((int64_t)(m0 + g) * K + k0);
    } else {
      // The last row tile: rows past M read row M - 1.
      const int gb = m0 + g < M ? m0 + g : M - 1;
      const int r = m0 + g + dl.lrow < M ? m0 + g + dl.lrow : M - 1;
      voff = (uint32_t)((r - gb) * K * 2) + dl.cb(i);
      return X + ((int64_t)gb * K + k0);
    }
  };
  tile_kloop<E>(K, lds, acc, wrow, xrow);

  // Epilogue through LDS (every wave is past its last LDS read at the barrier).
  wait_lgkm0();
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int nb = 0; nb < kWB; ++nb)
#pragma unroll
    for (int mb = 0; mb < kXB; ++mb) {
      const int ml = wm * 64 + mb * 16 + rl;
      const int nl = wn * 128 + nb * 16 + 4 * q;
      const floatx4& v = acc[nb][mb];
      const u32x2 pk = {pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
      *(u32x2*)(lds + ml * 512 + ((nl >> 3) ^ (ml & 31)) * 16 + (nl & 7) * 2) = pk;
    }
  wait_lgkm0();
  __builtin_amdgcn_s_barrier();
  const int hi = lane >> 5;
  const int l32 = lane & 31;
#pragma unroll
  for (int i = 0; i < kGT / 16; ++i) {
    const int row = (i * 8 + wave) * 2 + hi;
    const u32x4 v = *(const u32x4*)(lds + row * 512 + ((l32 ^ (row & 31)) * 16));
    if (FULL_M || m0 + row < M)
      __builtin_nontemporal_store(v, (u32x4*)(C + (int64_t)(m0 + row) * N + n0 + l32 * 8));
  }
}

template <typename T>
__global__ __launch_bounds__(kGThreads) void gemm_nt_kernel(const uint16_t* __restrict__ X,
                                                             const uint16_t* __restrict__ W,
                                                             uint16_t* __restrict__ C, int M,
                                                             int N, int K) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int mt = (M + kGT - 1) / kGT;
  const int m0 = (int)(blockIdx.x % mt) * kGT;
  const int n0 = (int)(blockIdx.x / mt) * kGT;
  if (m0 + kGT <= M)
    gemm_tile<T, true>(X, W, C, M, N, K, m0, n0, lds);
  else
    gemm_tile<T, false>(X, W, C, M, N, K, m0, n0, lds);
}

}  // namespace
}  // namespace mqc

using namespace mqc;

namespace {
constexpr int kMaxDevices = 64;
std::atomic<bool> g_lds_attr_set[kMaxDevices];
}  // namespace

extern "C" {

int mqc_gemm_nt(const void* X, const void* W, void* C, int64_t M, int64_t N, int64_t K, int dtype,
                void* stream) {
  if (M < 0 || N < 0 || K < 0) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  if (dtype == MQC_F32) return MQC_E_DTYPE;  // 16-bit MFMAs only
  if (M == 0 || N == 0) return MQC_OK;
  if (K == 0 || N % kGT != 0 || K % kGBK != 0) return MQC_E_SHAPE;
  if (!X || !W || !C) return MQC_E_NULL;
  if (!aligned(X, 16) || !aligned(W, 16) || !aligned(C, 16)) return MQC_E_ALIGN;
  // 32-bit tile and row arithmetic.
  if (M > (1LL << 30) || N > (1LL << 30) || K > (1LL << 20)) return MQC_E_LIMIT;
  const int64_t tiles = (M + kGT - 1) / kGT * (N / kGT);
  if (tiles > 0x7fffffffLL) return MQC_E_LIMIT;
  // The LDS limit is a per-device attribute of the kernel: set once on each
  // device (idempotent, so two threads racing only repeat the call).
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return MQC_E_LIMIT;
  if (!g_lds_attr_set[dev].load(std::memory_order_acquire)) {
    e = hipFuncSetAttribute((const void*)gemm_nt_kernel<bf16_t>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e == hipSuccess)
      e = hipFuncSetAttribute((const void*)gemm_nt_kernel<f16_t>,
                              hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return (int)e;
    g_lds_attr_set[dev].store(true, std::memory_order_release);
  }
  if (dtype == MQC_BF16)
    hipLaunchKernelGGL(gemm_nt_kernel<bf16_t>, dim3((unsigned)tiles), dim3(kGThreads), kLdsBytes,
                       (hipStream_t)stream, (const uint16_t*)X, (const uint16_t*)W, (uint16_t*)C,
                       (int)M, (int)N, (int)K);
  else
    hipLaunchKernelGGL(gemm_nt_kernel<f16_t>, dim3((unsigned)tiles), dim3(kGThreads), kLdsBytes,
                       (hipStream_t)stream, (const uint16_t*)X, (const uint16_t*)W, (uint16_t*)C,
                       (int)M, (int)N, (int)K);
  return launch_status();
}

}  // extern "C"
