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
//   - 256 x 256 output tile per workgroup of 8 waves (two per SIMD); wave w owns 128 columns
//     (w >> 2) x 64 rows (w & 3) as 8 x 4 blocks of v_mfma_f32_16x16x32_bf16 accumulators
//     (128 fp32 per lane). W rows are the MFMA's first operand and X rows its second, so
//     each lane ends with 4 consecutive output columns of one row per 16 x 16 block. On
//     random operands the 16 x 16 x 32 shape sustains more than the 32 x 32 x 16 one:
//     measured with operands held in registers, 2098 against 1785 TFLOP/s (both about
//     2400 on zeros: the MFMA rate depends on the operand data through the chip's power).
//   - K in steps of 64 through two LDS stages of 64 KB (X and W tiles of 256 rows x 128
//     bytes), filled by global_load_lds_dwordx4 (16 bytes per lane straight into LDS) in its
//     scalar-base form: each DMA instruction covers 8 rows whose base address is
//     wave-uniform (SGPRs), and a lane adds one of two 32-bit offsets (the swizzle below
//     depends on the row group's parity only), so the loads take 2 VGPRs instead of a
//     64-bit pointer per instruction. The 16-byte chunk c of row r is stored at chunk
//     c ^ ((r >> 1) & 7), so the 16 rows one ds_read_b128 group reads fall on distinct banks.
//   - One barrier per K step: after it, the stage consumed before it is free and receives
//     the loads of the next step, which then run during this step's MFMAs. The fragments
//     of the step's second K slice are read while the first slice's MFMAs issue, one read
//     after each MFMA.
//   - Tiles in launch order with the M tile fastest: the 256 tiles in flight cover all of X
//     (in the Infinity Cache) and a few W tiles, each of which is read from HBM about once.
//   - Epilogue through LDS: the tile is written to LDS in the MFMA layout (rows of 512 bytes,
//     16-byte chunks XORed with row & 31) and read back as whole rows, so every global
//     store writes 16 bytes per lane along a row (nontemporal: C is not read back here).
// Rows of X past M are clamped onto row M - 1 for the loads and never stored, so M is
// free; N must be a multiple of 256 and K of 64.
#include <atomic>

#include "common.hpp"

namespace mqc {
namespace {

typedef __bf16 gbf16x8 __attribute__((ext_vector_type(8)));
typedef float gfloatx4 __attribute__((ext_vector_type(4)));
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
constexpr int kWB = 8;                     // 16-row W blocks per wave
constexpr int kXB = 4;                     // 16-row X blocks per wave

// 16 bytes per lane from global memory (sbase + voff, sbase wave-uniform) into LDS at
// lds_addr + lane * 16. The kernel waits for these with explicit s_waitcnt vmcnt; issued
// as inline assembly because the compiler, unable to tell the two stages apart, would
// otherwise wait for every load in flight before each LDS read. M0 is set here; nothing
// else in this kernel uses it.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // M0 in the clobber list, as intended
__device__ inline void dma16(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(sbase), "s"(lds_addr) : "memory", "m0");
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

// One 256 x 256 tile. FULL_M: all 256 rows of the tile exist (every row tile but a
// ragged last one, whose rows past M read row M - 1).
template <bool FULL_M>
__device__ inline void gemm_tile(const __bf16* __restrict__ X, const __bf16* __restrict__ W,
                                 __bf16* __restrict__ C, int M, int N, int K, int m0, int n0,
                                 char* lds) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // DMA instruction i of this wave carries tile rows (wave * kLoads + i) * 8 + lrow, lane
  // chunk (lane % 8) ^ swizzle; the swizzle depends on the parity of i only.
  const int lrow = lane >> 3;
  const int lslot = lane & 7;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void_t*)lds;
  uint32_t voff[2], cbyte[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    cbyte[p] = (uint32_t)((lslot ^ ((p * 4 + (lrow >> 1)) & 7)) * 16);
    voff[p] = (uint32_t)(lrow * K * 2) + cbyte[p];
  }
  auto issue_stage = [&](int kt) {
    const int k0 = kt * kGBK;
    const uint32_t sb = lds0 + (uint32_t)((kt & 1) * kStageBytes);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int g = (wave * kLoads + i) * kRowsPerLoad;
      const uint32_t off = (uint32_t)((wave * kLoads + i) * 1024);
      dma16(W + ((int64_t)(n0 + g) * K + k0), voff[i & 1], sb + off);
      if constexpr (FULL_M) {
        dma16(X + ((int64_t)(m0 + g) * K + k0), voff[i & 1], sb + kTileBytes + off);
      } else {
        // The last row tile: rows past M read row M - 1.
        const int gb = m0 + g < M ? m0 + g : M - 1;
        const int r = m0 + g + lrow < M ? m0 + g + lrow : M - 1;
        dma16(X + ((int64_t)gb * K + k0), (uint32_t)((r - gb) * K * 2) + cbyte[i & 1],
              sb + kTileBytes + off);
      }
    }
  };

  const int wn = wave >> 2;
  const int wm = wave & 3;
  const int rl = lane & 15;  // row within a 16-row block
  const int q = lane >> 4;   // 16-byte chunk within a 32-wide K slice
  gfloatx4 acc[kWB][kXB];
#pragma unroll
  for (int a = 0; a < kWB; ++a)
#pragma unroll
    for (int b = 0; b < kXB; ++b) acc[a][b] = (gfloatx4){};
  // LDS byte offsets of this lane's fragments per K slice; the blocks of a wave are
  // 16 rows apart, which keeps the swizzle, so they add constants.
  int woff[2], xoff[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const int c = 4 * kk + q;
    const int rw = wn * 128 + rl;
    woff[kk] = rw * kRowBytes + gswz(rw, c) * 16;
    const int rx = wm * 64 + rl;
    xoff[kk] = kTileBytes + rx * kRowBytes + gswz(rx, c) * 16;
  }
  gbf16x8 wf[2][kWB], xf[2][kXB];
  auto read_frags = [&](int buf, const char* sb, int kk) {
#pragma unroll
    for (int nb = 0; nb < kWB; ++nb) wf[buf][nb] = *(const gbf16x8*)(sb + woff[kk] + nb * 16 * kRowBytes);
#pragma unroll
    for (int mb = 0; mb < kXB; ++mb) xf[buf][mb] = *(const gbf16x8*)(sb + xoff[kk] + mb * 16 * kRowBytes);
  };
  auto mfmas = [&](int buf) {
#pragma unroll
    for (int nb = 0; nb < kWB; ++nb)
#pragma unroll
      for (int mb = 0; mb < kXB; ++mb)
        acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[buf][nb], xf[buf][mb], acc[nb][mb], 0, 0, 0);
  };

  const int KT = K / kGBK;
  issue_stage(0);
  for (int kt = 0; kt < KT; ++kt) {
    // This wave's loads of stage kt are the only ones in flight.
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (kt + 1 < KT) issue_stage(kt + 1);
    const char* sbase = lds + (kt & 1) * kStageBytes;
    read_frags(0, sbase, 0);
    __builtin_amdgcn_sched_barrier(0);
    // First K slice: its MFMAs with the second slice's fragment reads, one after each MFMA.
    read_frags(1, sbase, 1);
    mfmas(0);
#pragma unroll
    for (int g = 0; g < kWB + kXB; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    __builtin_amdgcn_sched_barrier(0);
    mfmas(1);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Epilogue through LDS (every wave is past its last LDS read at the barrier).
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int nb = 0; nb < kWB; ++nb)
#pragma unroll
    for (int mb = 0; mb < kXB; ++mb) {
      const int ml = wm * 64 + mb * 16 + rl;
      const int nl = wn * 128 + nb * 16 + 4 * q;
      const gfloatx4& v = acc[nb][mb];
      const gu32x2 pk = {pk_bf16(v[0], v[1]), pk_bf16(v[2], v[3])};
      *(gu32x2*)(lds + ml * 512 + ((nl >> 3) ^ (ml & 31)) * 16 + (nl & 7) * 2) = pk;
    }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  const int hi = lane >> 5;
  const int l32 = lane & 31;
#pragma unroll
  for (int i = 0; i < kGT / 16; ++i) {
    const int row = (i * 8 + wave) * 2 + hi;
    const gu32x4 v = *(const gu32x4*)(lds + row * 512 + ((l32 ^ (row & 31)) * 16));
    if (FULL_M || m0 + row < M)
      __builtin_nontemporal_store(v, (gu32x4*)(C + (int64_t)(m0 + row) * N + n0 + l32 * 8));
  }
}

__global__ __launch_bounds__(kGThreads) void gemm_nt_bf16_kernel(const __bf16* __restrict__ X,
                                                                  const __bf16* __restrict__ W,
                                                                  __bf16* __restrict__ C, int M,
                                                                  int N, int K) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int mt = (M + kGT - 1) / kGT;
  const int m0 = (int)(blockIdx.x % mt) * kGT;
  const int n0 = (int)(blockIdx.x / mt) * kGT;
  if (m0 + kGT <= M)
    gemm_tile<true>(X, W, C, M, N, K, m0, n0, lds);
  else
    gemm_tile<false>(X, W, C, M, N, K, m0, n0, lds);
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
