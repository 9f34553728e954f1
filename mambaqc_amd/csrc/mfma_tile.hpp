#pragma once
// The MFMA main loop shared by the library's 16-bit GEMM tiles (gfx950; bf16 or fp16
// operands, E = __bf16 or _Float16):
//   acc += W_tile[TW rows, K] . X_tile[TX rows, K]^T
// for one output tile, fp32 accumulation. Described here for the 256 x 256 tile of the
// projections (Tile256); TileCfg gives smaller tiles the same loop.
//
//   - 8 waves (two per SIMD); wave w owns W rows (w >> 2) * 128 + [0, 128) and X rows
//     (w & 3) * 64 + [0, 64) as 8 x 4 blocks of v_mfma_f32_16x16x32_bf16 (_f16) accumulators
//     (128 fp32 per lane). W rows are the MFMA's first operand and X rows its second, so
//     in block (nb, mb) lane l holds the 4 consecutive W rows
//     (w >> 2) * 128 + nb * 16 + 4 * (l >> 4) + [0, 4) of X row (w & 3) * 64 + mb * 16 +
//     (l & 15). On random operands the 16 x 16 x 32 shape sustains more than the
//     32 x 32 x 16 one: measured with operands held in registers, 2098 against
//     1785 TFLOP/s (both about 2400 on zeros: the MFMA rate depends on the operand data
//     through the chip's power).
//   - K in steps of 64 through two LDS stages of 64 KB (X and W tiles of 256 rows x 128
//     bytes), filled by global_load_lds_dwordx4 (16 bytes per lane straight into LDS) in
//     its scalar-base form: each DMA instruction covers 8 rows whose base address is
//     wave-uniform (SGPRs), and a lane adds a 32-bit offset, so the loads take one VGPR
//     each instead of a 64-bit pointer. The 16-byte chunk c of row r is stored at chunk
//     c ^ ((r >> 1) & 7), so the 16 rows one ds_read_b128 group reads fall on distinct
//     banks.
//   - One barrier per K step: after it, the stage consumed before it is free and receives
//     the loads of the next step, which then run during this step's MFMAs. The fragments
//     of the step's second K slice are read while the first slice's MFMAs issue, one read
//     after each MFMA.
#include "common.hpp"

namespace mqc {
namespace mfma {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kT = 256;                   // tile rows and columns
constexpr int kBK = 64;                   // K per stage
constexpr int kThreads = 512;             // 8 waves
constexpr int kRowBytes = kBK * 2;        // 128 bytes of a tile row per stage
constexpr int kTileBytes = kT * kRowBytes;     // 32 KB
constexpr int kStageBytes = 2 * kTileBytes;    // X and W tiles
constexpr int kStagesBytes = 2 * kStageBytes;  // two stages = 128 KB
constexpr int kRowsPerLoad = 64 * 16 / kRowBytes;  // 8 rows per DMA instruction
constexpr int kLoads = kT / kRowsPerLoad / 8;      // 4 per wave per operand per stage
constexpr int kWB = 8;                    // 16-row W blocks per wave
constexpr int kXB = 4;                    // 16-row X blocks per wave

// 16 bytes per lane from global memory (sbase + voff, sbase wave-uniform) into LDS at
// lds_addr + lane * 16. The kernel waits for these with explicit s_waitcnt vmcnt; issued
// as inline assembly because the compiler, unable to tell the two stages apart, would
// otherwise wait for every load in flight before each LDS read. M0 is set here; nothing
// else in these kernels uses it.
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

// One 16 x 16 x 32 MFMA of 16-bit operands into fp32, by operand type.
__device__ inline floatx4 mfma16(const bf16x8& a, const bf16x8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ inline floatx4 mfma16(const f16x8& a, const f16x8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
template <typename E> struct FragOf;
template <> struct FragOf<__bf16> { using type = bf16x8; };
template <> struct FragOf<_Float16> { using type = f16x8; };

// s_waitcnt vmcnt(N) with expcnt and lgkmcnt at their maxima (gfx9 fields).
template <int N>
__device__ inline void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(0) (LDS and scalar memory) with vmcnt and expcnt at their maxima.
__device__ inline void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Per-lane DMA geometry: DMA instruction i of a wave carries tile rows
// (wave * kLoads + i) * 8 + lrow(), 16-byte chunk lslot() ^ swizzle; the swizzle
// depends on the parity of i only, so a lane needs two chunk offsets.
struct DmaLane {
  int lrow;
  uint32_t cbyte[2];
  __device__ explicit DmaLane(int lane) : lrow(lane >> 3) {
    const int lslot = lane & 7;
#pragma unroll
    for (int p = 0; p < 2; ++p) cbyte[p] = (uint32_t)((lslot ^ ((p * 4 + (lrow >> 1)) & 7)) * 16);
  }
  // The chunk offset of DMA group i (selected: i may be a wave-dependent value, and an
  // indexed register array would go to scratch).
  __device__ uint32_t cb(int i) const { return (i & 1) ? cbyte[1] : cbyte[0]; }
};

// Tile shape: TW rows of W by TX rows of X, NW_W x NW_X waves (wave w owns W rows
// (w / NW_X) * (TW / NW_W) + [0, TW / NW_W) and X rows (w % NW_X) * (TX / NW_X) + [0, TX / NW_X)
// as WB x XB blocks of 16 x 16 accumulators). Every DMA instruction carries 8 rows of one
// operand; a wave issues TW / 8 / waves of them for W and TX / 8 / waves for X per stage.
template <int TW_, int TX_, int NW_W_, int NW_X_>
struct TileCfg {
  static constexpr int TW = TW_, TX = TX_, NW_W = NW_W_, NW_X = NW_X_;
  static constexpr int kWaves = NW_W * NW_X;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int WB = TW / NW_W / 16;
  static constexpr int XB = TX / NW_X / 16;
  static constexpr int kWBytes = TW * kRowBytes;              // W tile of one stage
  static constexpr int kStageBytes = (TW + TX) * kRowBytes;
  static constexpr int kStagesBytes = 2 * kStageBytes;
  static constexpr int kWLoads = TW / kRowsPerLoad / kWaves;  // DMA instructions per wave
  static constexpr int kXLoads = TX / kRowsPerLoad / kWaves;
  static_assert(TW % (16 * NW_W) == 0 && TX % (16 * NW_X) == 0, "whole 16-row blocks");
  static_assert(TW % (kRowsPerLoad * kWaves) == 0 && TX % (kRowsPerLoad * kWaves) == 0,
                "whole DMA groups per wave");
};

// The library's 256 x 256 tile (8 waves of 128 W rows x 64 X rows).
using Tile256 = TileCfg<kT, kT, 2, 4>;
static_assert(Tile256::WB == kWB && Tile256::XB == kXB && Tile256::kStagesBytes == kStagesBytes,
              "the 256 x 256 constants above");

// The K loop of one tile into acc (which it does not clear). For DMA instruction i of
// this wave (tile rows g .. g + 7 of one operand) and K offset k0 (in elements):
//   wrow(g, k0, i, voff, dl), xrow(g, k0, i, voff, dl)
//       -> a wave-uniform pointer for W's (X's) rows g .. g + 7 at column k0, with the
//          lane's byte offset from it written to voff: lane row dl.lrow, 16-byte chunk
//          dl.cb(i) (i the operand's DMA group index, whose parity sets the
//          swizzle), row pitch ld * 2 bytes; the caller may clamp rows past the matrix.
// Returns after the last MFMA; the caller waits on lgkmcnt and barriers before reusing
// the LDS stages.
// LDS address of the dynamic LDS array (for the DMA's M0).
__device__ inline uint32_t lds_addr(char* lds) { return (uint32_t)(uintptr_t)(lds_void_t*)lds; }

// The DMA of K stage kt (into LDS stage kt & 1) for the K loop below; wave is the
// (wave-uniform) wave index, dl the lane's DmaLane and lds0 = lds_addr(lds).
template <typename Cfg, typename WRow, typename XRow>
__device__ inline void tile_issue_stage(int kt, int wave, uint32_t lds0, const DmaLane& dl,
                                        const WRow& wrow, const XRow& xrow) {
  const int k0 = kt * kBK;
  const uint32_t sb = lds0 + (uint32_t)((kt & 1) * Cfg::kStageBytes);
  constexpr int NL = Cfg::kWLoads > Cfg::kXLoads ? Cfg::kWLoads : Cfg::kXLoads;
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    if (i < Cfg::kWLoads) {
      const int gi = wave * Cfg::kWLoads + i;
      uint32_t wv;
      const void* wb = wrow(gi * kRowsPerLoad, k0, gi, wv, dl);
      dma16(wb, wv, sb + (uint32_t)(gi * 1024));
    }
    if (i < Cfg::kXLoads) {
      const int gi = wave * Cfg::kXLoads + i;
      uint32_t xv;
      const void* xb = xrow(gi * kRowsPerLoad, k0, gi, xv, dl);
      dma16(xb, xv, sb + (uint32_t)(Cfg::kWBytes + gi * 1024));
    }
  }
}

template <typename Cfg, typename E = __bf16, typename WRow, typename XRow>
__device__ inline void tile_kloop_cfg(int K, char* lds,
                                      floatx4 (&acc)[Cfg::WB][Cfg::XB], const WRow& wrow,
                                      const XRow& xrow) {
  constexpr int WB = Cfg::WB, XB = Cfg::XB;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const DmaLane dl(lane);
  const uint32_t lds0 = lds_addr(lds);
  auto issue_stage = [&](int kt) { tile_issue_stage<Cfg>(kt, wave, lds0, dl, wrow, xrow); };

  const int wn = wave / Cfg::NW_X;
  const int wm = wave % Cfg::NW_X;
  const int rl = lane & 15;  // row within a 16-row block
  const int q = lane >> 4;   // 16-byte chunk within a 32-wide K slice
  // LDS byte offsets of this lane's fragments per K slice; the blocks of a wave are
  // 16 rows apart, which keeps the swizzle, so they add constants.
  int woff[2], xoff[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const int c = 4 * kk + q;
    const int rw = wn * (Cfg::TW / Cfg::NW_W) + rl;
    woff[kk] = rw * kRowBytes + gswz(rw, c) * 16;
    const int rx = wm * (Cfg::TX / Cfg::NW_X) + rl;
    xoff[kk] = Cfg::kWBytes + rx * kRowBytes + gswz(rx, c) * 16;
  }
  using frag = typename FragOf<E>::type;
  frag wf[2][WB], xf[2][XB];
  auto read_frags = [&](int buf, const char* sb, int kk) {
#pragma unroll
    for (int nb = 0; nb < WB; ++nb) wf[buf][nb] = *(const frag*)(sb + woff[kk] + nb * 16 * kRowBytes);
#pragma unroll
    for (int mb = 0; mb < XB; ++mb) xf[buf][mb] = *(const frag*)(sb + xoff[kk] + mb * 16 * kRowBytes);
  };
  auto mfmas = [&](int buf) {
#pragma unroll
    for (int nb = 0; nb < WB; ++nb)
#pragma unroll
      for (int mb = 0; mb < XB; ++mb)
        acc[nb][mb] = mfma16(wf[buf][nb], xf[buf][mb], acc[nb][mb]);
  };

  const int KT = K / kBK;
  issue_stage(0);
  for (int kt = 0; kt < KT; ++kt) {
    // This wave's loads of stage kt are the only ones in flight.
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (kt + 1 < KT) issue_stage(kt + 1);
    const char* sbase = lds + (kt & 1) * Cfg::kStageBytes;
    read_frags(0, sbase, 0);
    __builtin_amdgcn_sched_barrier(0);
    // First K slice: its MFMAs with the second slice's fragment reads, one after each MFMA.
    read_frags(1, sbase, 1);
    mfmas(0);
#pragma unroll
    for (int g = 0; g < WB + XB; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    __builtin_amdgcn_sched_barrier(0);
    mfmas(1);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The 256 x 256 tile's K loop (E: the operands' 16-bit type).
template <typename E = __bf16, typename WRow, typename XRow>
__device__ inline void tile_kloop(int K, char* lds, floatx4 (&acc)[kWB][kXB], const WRow& wrow,
                                  const XRow& xrow) {
  tile_kloop_cfg<Tile256, E>(K, lds, acc, wrow, xrow);
}

}  // namespace mfma
}  // namespace mqc
