// The block's output step in one launch (bf16): the quaternion -> real projection
// out_proj and the gated residual,
//   out[m, n] = x[m, n] + sigmoid(z[m, n]) * bf16(sum_k y[m, k] W[n, k] + bias[n])
// (QuaternionLinear._forward_quaternion_to_real, mambaqc/layers/quaternion_linear.py:163-172,
// called at mambaqc/models/quaternion_mamba2_block.py:157; the gate and residual at
// :160-164, with z[..., :d_model] as in the Lite block, quaternion_mamba2_lite_block.py:163).
// y is the QuaternionLayerNorm output viewed as [rows, 4 * d_inner] (quaternion components
// innermost, the reference's reshape), W the out_proj weight [d_model, 4 * d_inner].
//
// Unfused, the projection (hipBLASLt) writes y_real [rows, d_model] in bf16 and a second
// kernel reads it back with x and z. Here the GEMM's epilogue does the gate: y_real is
// rounded to bf16 as the projection would store it and never leaves the chip.
//
// Tiles: 128 tokens x 96 outputs (d_model 768 = 8 x 96, so batch 4 x 2048 tokens make 512
// tiles, two per CU), 4 waves of 64 tokens x 48 outputs, K in 64-wide stages through the
// MFMA main loop of mfma_tile.hpp (56 KiB of LDS: two workgroups share a CU). The tile
// order gives each XCD a contiguous range of tiles, the outputs of a token tile adjacent,
// so the tiles that read the same rows of y share an L2. Epilogue: the tile, rounded to
// bf16, through LDS (rows padded to 208 bytes against bank conflicts) and back as
// 16-byte pieces of rows, each gated against 16-byte pieces of x and z.
#include <atomic>

#include "mfma_tile.hpp"

namespace mqc {
namespace {

using namespace mfma;

using OutCfg = TileCfg<96, 128, 2, 2>;
constexpr int kON = OutCfg::TW;   // outputs per tile
constexpr int kOM = OutCfg::TX;   // tokens per tile
constexpr int kOThreads = OutCfg::kThreads;
constexpr int kOPitch = 208;      // bytes per staged row (96 bf16 = 192, padded)
constexpr int kOLds = OutCfg::kStagesBytes;
static_assert(kOM * kOPitch <= kOLds, "the staged tile fits the stages");

struct OutArgs {
  const __bf16* y;     // [M, K]
  const __bf16* w;     // [N, K]
  const __bf16* bias;  // [N] or null
  const __bf16* x;     // [M, N]
  const __bf16* z;     // [M, zs]
  __bf16* out;         // [M, N]
  int M, N, K;
  int64_t zs;
};

__device__ inline float bf2f(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

__global__ __launch_bounds__(kOThreads) void out_proj_gate_kernel(OutArgs a) {
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave / OutCfg::NW_X;
  const int wm = wave % OutCfg::NW_X;
  const int rl = lane & 15;
  const int q = lane >> 4;

  const int nt = (a.N + kON - 1) / kON;
  const int ntiles = (int)gridDim.x;
  const int lin = (int)blockIdx.x;
  const int logical = ntiles % kXCDs ? lin : (lin % kXCDs) * (ntiles / kXCDs) + lin / kXCDs;
  const int m0 = (logical / nt) * kOM;
  const int n0 = (logical % nt) * kON;
  const int K = a.K;

  floatx4 acc[OutCfg::WB][OutCfg::XB];
#pragma unroll
  for (int i = 0; i < OutCfg::WB; ++i)
#pragma unroll
    for (int j = 0; j < OutCfg::XB; ++j) acc[i][j] = (floatx4){};
  // Rows past the matrix (a ragged last token or output tile) read its last row and are
  // never stored.
  auto rows = [&](const __bf16* base, int r0, int rmax, int g, int k0, int i, uint32_t& voff,
                  const DmaLane& dl) -> const void* {
    const int gb = r0 + g < rmax ? r0 + g : rmax - 1;
    const int r = r0 + g + dl.lrow < rmax ? r0 + g + dl.lrow : rmax - 1;
    voff = (uint32_t)((r - gb) * K * 2) + dl.cb(i);
    return base + ((int64_t)gb * K + k0);
  };
  auto wrow = [&](int g, int k0, int i, uint32_t& voff, const DmaLane& dl) -> const void* {
    return rows(a.w, n0, a.N, g, k0, i, voff, dl);
  };
  auto xrow = [&](int g, int k0, int i, uint32_t& voff, const DmaLane& dl) -> const void* {
    return rows(a.y, m0, a.M, g, k0, i, voff, dl);
  };
  tile_kloop_cfg<OutCfg>(K, lds, acc, wrow, xrow);

  // The projection's tile, + bias, rounded to bf16, staged as [token][output].
  wait_lgkm0();
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int nb = 0; nb < OutCfg::WB; ++nb) {
    const int nl = wn * (kON / OutCfg::NW_W) + nb * 16 + 4 * q;
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.bias) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int n = n0 + nl + e < a.N ? n0 + nl + e : a.N - 1;
        bv[e] = (float)a.bias[n];
      }
    }
#pragma unroll
    for (int mb = 0; mb < OutCfg::XB; ++mb) {
      const int ml = wm * (kOM / OutCfg::NW_X) + mb * 16 + rl;
      const floatx4& v = acc[nb][mb];
      const u32x2 pk = {pk_bf16(v[0] + bv[0], v[1] + bv[1]), pk_bf16(v[2] + bv[2], v[3] + bv[3])};
      *(u32x2*)(lds + ml * kOPitch + nl * 2) = pk;
    }
  }
  wait_lgkm0();
  __builtin_amdgcn_s_barrier();
  // Gate: 16-byte pieces (8 outputs) of staged rows; N is a multiple of 8.
  constexpr int kPieces = kOM * (kON / 8);
#pragma unroll
  for (int i = 0; i < kPieces / kOThreads; ++i) {
    const int c = tid + i * kOThreads;
    const int ml = c / (kON / 8);
    const int nl = (c - ml * (kON / 8)) * 8;
    const int m = m0 + ml;
    const int n = n0 + nl;
    if (m < a.M && n < a.N) {
      const u32x4 yv = *(const u32x4*)(lds + ml * kOPitch + nl * 2);
      const u32x4 xv = *(const u32x4*)(a.x + (int64_t)m * a.N + n);
      const u32x4 zv = *(const u32x4*)(a.z + (int64_t)m * a.zs + n);
      u32x4 o;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        float r[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t sh = 16 * h;
          const float g = 1.f / (1.f + __expf(-bf2f((zv[w] >> sh) & 0xffffu)));
          r[h] = fmaf(g, bf2f((yv[w] >> sh) & 0xffffu), bf2f((xv[w] >> sh) & 0xffffu));
        }
        o[w] = pk_bf16(r[0], r[1]);
      }
      *(u32x4*)(a.out + (int64_t)m * a.N + n) = o;
    }
  }
}

}  // namespace
}  // namespace mqc

using namespace mqc;

namespace {
constexpr int kMaxDevices = 64;
std::atomic<bool> g_out_attr_set[kMaxDevices];
}  // namespace

extern "C" {

int mqc_out_proj_gate_fwd(const void* y, const void* W, const void* bias, const void* x,
                          const void* z, int64_t z_row_stride, void* out, int64_t rows,
                          int64_t d_model, int64_t k, int dtype, void* stream) {
  if (rows < 0 || d_model < 0 || k < 0 || z_row_stride < 0) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  if (dtype != MQC_BF16) return MQC_E_DTYPE;  // bf16 MFMAs only
  if (rows == 0 || d_model == 0) return MQC_OK;
  if (k == 0 || k % kBK != 0 || d_model % 8 != 0 || z_row_stride < d_model ||
      z_row_stride % 8 != 0)
    return MQC_E_SHAPE;
  if (!y || !W || !x || !z || !out) return MQC_E_NULL;
  if (!aligned(y, 16) || !aligned(W, 16) || !aligned(x, 16) || !aligned(z, 16) ||
      !aligned(out, 16) || (bias && !aligned(bias, 2)))
    return MQC_E_ALIGN;
  // 32-bit tile and row arithmetic.
  if (rows > (1LL << 30) || d_model > (1LL << 20) || k > (1LL << 20) ||
      z_row_stride > (1LL << 32))
    return MQC_E_LIMIT;
  const int64_t tiles = (rows + kOM - 1) / kOM * ((d_model + kON - 1) / kON);
  if (tiles > 0x7fffffffLL) return MQC_E_LIMIT;
  // Tiles write out while other tiles still read y, W, bias and z. out may be x itself
  // (each 16-byte piece of x is read and then written by one thread), not a shifted x.
  const int64_t out_bytes = rows * d_model * 2;
  if (overlaps(out, out_bytes, y, rows * k * 2) || overlaps(out, out_bytes, W, d_model * k * 2) ||
      overlaps(out, out_bytes, bias, bias ? d_model * 2 : 0) ||
      overlaps(out, out_bytes, z, ((rows - 1) * z_row_stride + d_model) * 2) ||
      partial_overlap(out, x, out_bytes))
    return MQC_E_OVERLAP;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return MQC_E_LIMIT;
  if (!g_out_attr_set[dev].load(std::memory_order_acquire)) {
    e = hipFuncSetAttribute((const void*)out_proj_gate_kernel,
                            hipFuncAttributeMaxDynamicSharedMemorySize, kOLds);
    if (e != hipSuccess) return (int)e;
    g_out_attr_set[dev].store(true, std::memory_order_release);
  }
  OutArgs a{};
  a.y = (const __bf16*)y; a.w = (const __bf16*)W; a.bias = (const __bf16*)bias;
  a.x = (const __bf16*)x; a.z = (const __bf16*)z; a.out = (__bf16*)out;
  a.M = (int)rows; a.N = (int)d_model; a.K = (int)k; a.zs = z_row_stride;
  hipLaunchKernelGGL(out_proj_gate_kernel, dim3((unsigned)tiles), dim3(kOThreads), kOLds,
                     (hipStream_t)stream, a);
  return launch_status();
}

}  // extern "C"
