// Hand-written MFMA GEMM for the block's B/C projections (bf16):
//   C[M, N] = X[M, K] . W[N, K]^T,  fp32 accumulation, bf16 output,
// the nn.Linear layout of mambaqc/layers/quaternion_linear.py:145-161
// (F.linear(x, W) for the real -> quaternion maps B_proj and C_proj,
// models/quaternion_mamba2_block.py:186-191).
//
// This is the first stage of fusing the projections with the SSM walk: a
// GEMM whose tile loop this library owns. It is exported and tested, and
// measured against hipBLASLt on the same shapes; the block keeps hipBLASLt,
// which is faster at the config-3 shape (M 8192, N 393216, K 1536).
//
// Tiling (gfx950):
//   - 256 x 256 output tile per workgroup of 8 waves (two per SIMD); wave w
//     owns 128 columns (w >> 2) x 64 rows (w & 3): 4 x 2 v_mfma_f32_32x32x16_bf16
//     accumulators, 128 fp32 per lane. W rows are the MFMA's first operand and
//     X rows its second, so each lane ends with 4 consecutive output columns of
//     one row per 32 x 32 block.
//   - K in steps of 64 through two LDS stages of 64 KB (X and W tiles of 256
//     rows x 128 bytes), filled by global_load_lds_dwordx4 (16 bytes per lane
//     straight into LDS). The 16-byte chunk c of row r is stored at chunk
//     c ^ ((r >> 1) & 7), so the 16 rows one ds_read_b128 group reads fall on
//     distinct banks (SQ_LDS_BANK_CONFLICT measured 0).
//   - One barrier per K step: after it, the stage consumed before it is free
//     and receives the loads of the next step, which then run during this
//     step's 32 MFMAs per wave.
//   - Tiles in launch order with the M tile fastest: the 256 tiles in flight
//     cover all of X (in the Infinity Cache) and a few W tiles, each of which
//     is read from HBM about once (measured 11.2 ms against 13.2 ms for 8 x 4
//     tile patches per XCD).
//   - Epilogue through LDS: the tile is written to LDS in the MFMA layout
//     (rows of 512 bytes, 16-byte chunks XORed with row & 31) and read back
//     as whole rows, so every global store writes 16 bytes per lane along a
//     row (measured 2.9 ms of 11.2 for direct 8-byte stores of the MFMA layout,
//     about 1 ms this way).
// Rows of X past M are clamped onto row M - 1 for the loads and never stored,
// so M is free; N must be a multiple of 256 and K of 64.
#include <atomic>

#include "common.hpp"

namespace mqc {
namespace {

typedef __bf16 gbf16x8 __attribute__((ext_vector_type(8)));
typedef float gfloatx16 __attribute__((ext_vector_type(16)));
typedef unsigned int gu32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int gu32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kGT = 256;                   // tile rows and columns
constexpr int kGBK = 64;                   // K per stage
constexpr int kGThreads = 512;             // 8 waves
constexpr int kRowBytes = kGBK * 2;        // 128 bytes of a tile row per stage
constexpr int kTileBytes = kGT * kRowBytes;    // 32 KB
constexpr int kStageBytes = 2 * kTileBytes;    // X and W tiles
constexpr int kLdsBytes = 2 * kStageBytes;     // two stages = 128 KB (also the epilogue tile)
constexpr int kRowsPerLoad = 64 * 16 / kRowBytes;        // 8 rows per DMA instruction
constexpr int kLoads = kGT / kRowsPerLoad / 8;           // 4 per wave per operand per stage

// 16 bytes per lane from global memory into LDS at lds_addr + lane * 16. The
// kernel waits for these with explicit s_waitcnt vmcnt; issued as inline
// assembly because the compiler, unable to tell the two stages apart, would
// otherwise wait for every load in flight before each LDS read. M0 is set
// here; nothing else in this kernel uses it.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // M0 in the clobber list, as intended
__device__ inline void dma16(const void* gptr, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :: "v"(gptr), "s"(lds_addr) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ inline int gswz(int row, int c) { return c ^ ((row >> 1) & 7); }

__device__ inline uint32_t pk_bf16(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 h16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, h16x2));
}

// s_waitcnt vmcnt(N) with expcnt and lgkmcnt at their maxima (gfx9 fields).
template <int N>
__device__ inline void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

__global__ __launch_bounds__(kGThreads) void gemm_nt_bf16_kernel(const __bf16* __restrict__ X,
                                                                  const __bf16* __restrict__ W,
                                                                  __bf16* __restrict__ C, int M,
                                                                  int N, int K) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int mt = (M + kGT - 1) / kGT;
  const int m0 = (int)(blockIdx.x % mt) * kGT;
  const int n0 = (int)(blockIdx.x / mt) * kGT;

  // DMA sources: lane l of load i carries row (wave * kLoads + i) * 8 + l / 8
  // of the tile, logical chunk (l % 8) ^ swizzle.
  const int lrow = lane >> 3;
  const int lslot = lane & 7;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)lds;
  const __bf16* gw[kLoads];
  const __bf16* gx[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int row = (wave * kLoads + i) * kRowsPerLoad + lrow;
    const int c = gswz(row, lslot);
    const int xr = m0 + row < M ? m0 + row : M - 1;
    gw[i] = W + (int64_t)(n0 + row) * K + c * 8;
    gx[i] = X + (int64_t)xr * K + c * 8;
  }
  auto issue_stage = [&](int kt) {
    const int k0 = kt * kGBK;
    const uint32_t sb = lds0 + (uint32_t)((kt & 1) * kStageBytes);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const uint32_t off = (uint32_t)((wave * kLoads + i) * 1024);
      dma16(gw[i] + k0, __builtin_amdgcn_readfirstlane(sb + off));
      dma16(gx[i] + k0, __builtin_amdgcn_readfirstlane(sb + kTileBytes + off));
    }
  };

  const int wn = wave >> 2;
  const int wm = wave & 3;
  const int hi = lane >> 5;
  const int l32 = lane & 31;
  gfloatx16 acc[4][2];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = (gfloatx16){};
  int woff[4][4], xoff[4][2];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int c = 2 * kk + hi;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int row = wn * 128 + nb * 32 + l32;
      woff[kk][nb] = row * kRowBytes + gswz(row, c) * 16;
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int row = wm * 64 + mb * 32 + l32;
      xoff[kk][mb] = kTileBytes + row * kRowBytes + gswz(row, c) * 16;
    }
  }

  const int KT = K / kGBK;
  issue_stage(0);
  for (int kt = 0; kt < KT; ++kt) {
    // This wave's loads of stage kt are the only ones in flight.
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (kt + 1 < KT) issue_stage(kt + 1);
    const char* sbase = lds + (kt & 1) * kStageBytes;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      gbf16x8 wf[4], xf[2];
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) wf[nb] = *(const gbf16x8*)(sbase + woff[kk][nb]);
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) xf[mb] = *(const gbf16x8*)(sbase + xoff[kk][mb]);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
          acc[nb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[nb], xf[mb], acc[nb][mb], 0, 0, 0);
    }
  }

  // Epilogue through LDS (every wave is past its last LDS read at the barrier).
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      const int ml = wm * 64 + mb * 32 + l32;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int nl = wn * 128 + nb * 32 + 8 * jj + 4 * hi;
        const gfloatx16& v = acc[nb][mb];
        const gu32x2 pk = {pk_bf16(v[jj * 4 + 0], v[jj * 4 + 1]), pk_bf16(v[jj * 4 + 2], v[jj * 4 + 3])};
        *(gu32x2*)(lds + ml * 512 + ((nl >> 3) ^ (ml & 31)) * 16 + (nl & 7) * 2) = pk;
      }
    }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int i = 0; i < kGT / 16; ++i) {
    const int row = (i * 8 + wave) * 2 + hi;
    const gu32x4 v = *(const gu32x4*)(lds + row * 512 + ((l32 ^ (row & 31)) * 16));
    if (m0 + row < M) *(gu32x4*)(C + (int64_t)(m0 + row) * N + n0 + l32 * 8) = v;
  }
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
  if (dtype != MQC_BF16) return MQC_E_DTYPE;  // bf16 only
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
    e = hipFuncSetAttribute((const void*)gemm_nt_bf16_kernel,
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return (int)e;
    g_lds_attr_set[dev].store(true, std::memory_order_release);
  }
  hipLaunchKernelGGL(gemm_nt_bf16_kernel, dim3((unsigned)tiles), dim3(kGThreads), kLdsBytes,
                     (hipStream_t)stream, (const __bf16*)X, (const __bf16*)W, (__bf16*)C, (int)M,
                     (int)N, (int)K);
  return launch_status();
}

}  // extern "C"
