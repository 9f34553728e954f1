// Skinny GEMM for the projections of the recurrent decode step (bf16 / fp16):
//   Y[M, N] = X[M, K] . W[N, K]^T (+ bias[N]),  M <= 16 rows, fp32 accumulation,
// the nn.Linear / F.linear layout of mambaqc/layers/quaternion_linear.py:145-172
// and of the block's nn.Linear layers (models/quaternion_mamba2_block.py:78-122)
// at the few token rows of one decode step. One launch can take a pair of
// weights that share X (dt_proj and gate_proj, B_proj and C_proj).
//
// A decode step reads every weight once and does almost no arithmetic, so each
// projection is a read of W at HBM speed, and the small ones are a launch each.
// The product runs on the MFMA unit, which leaves the VALU idle and needs no
// cross-lane reductions:
//   - one wave per tile of 16 weight rows; per K step of 32 it issues one
//     v_mfma_f32_16x16x32 with W's 16 rows as the B operand (lane l holds 8
//     consecutive k of row l % 16, straight from HBM, 16 bytes per lane) and
//     X as the A operand (row l % 16 from LDS; lanes past M hold zeros);
//   - K steps are loaded in groups of 8 (8 KB per wave in flight), with enough
//     waves per CU (small register and LDS footprint) to cover HBM latency;
//   - the 16 x 16 result lands as rows 4 (l / 16) + i of column l % 16; the
//     lanes holding rows < M add the bias and store them.
// X (M x K, at most 64 KB) is copied to LDS once per workgroup, rows padded by
// 16 bytes so the A reads of different rows fall on different banks. Rows of W
// past N are clamped onto row N - 1 for the loads and never stored.
//
// Weights with few rows would leave most CUs idle with one wave per tile, so
// then 4, 8 or 16 waves share each tile's K (see skinny_launch).
//
// Weights with many rows, at most 8 token rows and K a multiple of 64 take the
// wide mode instead (skinny_wide_kernel): a tile reads each weight row as 64
// bytes per instruction (half a 128-byte line), while the wide mode's load
// instructions read 8 whole lines each and keep all of a row group's lines in
// flight; its products run on the VALU as dot2 instructions.
//
// Measured on MI355X at 4 rows (bf16): a pair of [1024 x 1024] weights in one
// launch 6.3 us, where hipBLASLt takes about 6.6 us per weight; [131072 x 1024]
// pairs (the small preset's B/C) 95-98 us in tiles against 99.7 us for two
// calls. The wide mode, same box, pairs at 4 rows unless noted, against tiles
// and hipBLASLt: [131072 x 1024] 87-90 / 100-102 / 114-115 us; the base
// preset's [393216 x 1536] 386-392 / 424-425 / 427 us (6.2 TB/s), at 1 row
// 369-371 / 414-419 / 436, at 8 rows 415-416 / 455-457 / 452-458;
// [524288 x 2048] 688-690 / 746 / 878-888 us. Decode steps of 4 tokens with
// every projection here: base preset 5.73 -> 5.30 ms eager and 5.68-5.73 ->
// 5.29-5.30 ms as a HIP graph against the B/C pair on hipBLASLt (same box;
// earlier, moving the other projections here took 5.89 -> 5.72 ms), small
// preset 2.05 -> 1.37 ms eager and 1.27 -> 1.09 ms as a graph.
#include <atomic>

#include "common.hpp"

namespace mqc {
namespace {

typedef __bf16 skbf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 skf16x8 __attribute__((ext_vector_type(8)));
typedef float skfloatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int sku32x4 __attribute__((ext_vector_type(4)));

constexpr int kSkThreads = 256;
constexpr int kSkWaves = kSkThreads / 64;
constexpr int kSkMaxRows = 16;
constexpr int kSkStep = 32;  // K per MFMA
constexpr int kSkGroup = 8;  // K steps loaded together
constexpr int64_t kSkMaxLds = 64 << 10;  // X in LDS, plus the split modes' partial tiles
constexpr int kSkBlocksPerCU = 8;
constexpr int kSkCUs = 256;  // MI355X compute units

template <typename T> struct SkVec;
template <> struct SkVec<bf16_t> { using type = skbf16x8; };
template <> struct SkVec<f16_t> { using type = skf16x8; };

template <typename T>
__device__ inline skfloatx4 sk_mfma(typename SkVec<T>::type a, typename SkVec<T>::type b,
                                    skfloatx4 c) {
  if constexpr (std::is_same<T, bf16_t>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

struct SkArgs {
  const void* x;
  const void* w[2];
  const void* bias[2];  // or nullptr
  void* y[2];
  int64_t n[2];
  int64_t tiles0;  // 16-row tiles of the first weight
  int64_t tiles;   // of both
  int64_t groups0;  // 8-row groups of the first weight (wide mode)
  int64_t groups;   // of both
  int M, K;
};

// Elements per LDS row of X.
__host__ __device__ inline int64_t sk_lds_row(int64_t K) { return K + 8; }

// SPLIT = 1: each wave owns whole tiles (4 per workgroup). SPLIT = 4, 8 or 16:
// the workgroup's SPLIT waves share one tile, each summing a contiguous part
// of K, and the partial 16 x 16 tiles are added through LDS (for weights with
// few rows, which would otherwise leave most CUs idle).
template <typename T, int SPLIT>
__global__ __launch_bounds__(SPLIT == 1 ? kSkThreads : 64 * SPLIT) void skinny_nt_kernel(SkArgs a) {
  using V = typename SkVec<T>::type;
  constexpr int NT = SPLIT == 1 ? kSkThreads : 64 * SPLIT;
  constexpr int WPB = NT / 64;                      // waves per workgroup
  constexpr int TPB = SPLIT == 1 ? WPB : 1;         // tiles per workgroup
  extern __shared__ __align__(16) unsigned char sk_lds[];
  const int K = a.K;
  const int M = a.M;
  const int64_t ldsRow = sk_lds_row(K);
  float* red = (float*)(sk_lds + M * ldsRow * 2);   // SPLIT x 64 lanes x 4 partials
  {
    // X -> LDS, 16 bytes per thread and step (K % 32 == 0, X 16-byte aligned).
    const int per_row = K / 8;
    for (int i = threadIdx.x; i < M * per_row; i += NT) {
      const int r = i / per_row;
      const int c = i - r * per_row;
      *(uint4*)(sk_lds + (r * ldsRow + c * 8) * 2) =
          ((const uint4*)a.x)[(int64_t)r * per_row + c];
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int col = lane & 15;  // the A row (token) and the B column (weight row) of this lane
  const int grp = lane >> 4;  // which 8 of a step's 32 k this lane holds
  const bool arow = col < M;
  const unsigned char* xa = sk_lds + ((arow ? col : 0) * ldsRow + 8 * grp) * 2;
  const int steps = K / kSkStep;
  // This wave's K steps: all of them, or its share of the tile's.
  const int s_lo = SPLIT == 1 ? 0 : (int)((int64_t)steps * wave / SPLIT);
  const int s_hi = SPLIT == 1 ? steps : (int)((int64_t)steps * (wave + 1) / SPLIT);
  for (int64_t tile0 = (int64_t)blockIdx.x * TPB; tile0 < a.tiles;
       tile0 += (int64_t)gridDim.x * TPB) {
    const int64_t tile = tile0 + (SPLIT == 1 ? wave : 0);
    // (SPLIT == 1: a wave past the last tile has nothing to do; no barrier follows.)
    if (tile < a.tiles) {
      const int which = tile >= a.tiles0 ? 1 : 0;
      const int64_t t = tile - (which ? a.tiles0 : 0);
      const int64_t N = a.n[which];
      const int64_t n = t * 16 + col;
      const T* wp = (const T*)a.w[which] + (n < N ? n : N - 1) * K + 8 * grp;
      skfloatx4 acc = {0.f, 0.f, 0.f, 0.f};
      int s = s_lo;
      for (; s + kSkGroup <= s_hi; s += kSkGroup) {
        V b[kSkGroup];
#pragma unroll
        for (int u = 0; u < kSkGroup; ++u) b[u] = *(const V*)(wp + (s + u) * kSkStep);
#pragma unroll
        for (int u = 0; u < kSkGroup; ++u) {
          V av{};
          if (arow) av = *(const V*)(xa + (s + u) * kSkStep * 2);
          acc = sk_mfma<T>(av, b[u], acc);
        }
      }
      for (; s < s_hi; ++s) {
        const V b = *(const V*)(wp + s * kSkStep);
        V av{};
        if (arow) av = *(const V*)(xa + s * kSkStep * 2);
        acc = sk_mfma<T>(av, b, acc);
      }
      if constexpr (SPLIT > 1) {
        // Partial tiles through LDS; wave 0 adds them in wave order.
        *(skfloatx4*)(red + (wave * 64 + lane) * 4) = acc;
      }
      bool store = true;
      if constexpr (SPLIT > 1) {
        __syncthreads();
        store = wave == 0;
        if (store) {
          acc = *(const skfloatx4*)(red + lane * 4);
#pragma unroll
          for (int w = 1; w < SPLIT; ++w) acc += *(const skfloatx4*)(red + (w * 64 + lane) * 4);
        }
        __syncthreads();  // red is rewritten by the next tile
      }
      if (store && n < N) {
        const T* bp = (const T*)a.bias[which];
        const float bv = bp ? io<T>::to_f32(bp[n]) : 0.f;
        T* yp = (T*)a.y[which];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 4 * grp + i;
          if (m < M) yp[(int64_t)m * N + n] = io<T>::from_f32(acc[i] + bv);
        }
      }
    }
  }
}

// Wide mode. A wave takes 8 weight rows at a time; lane l reads row l / 8 and
// the 16 bytes at (l % 8) * 16 of each 128-byte line of it, so one load
// instruction covers 8 whole lines, and all K / 64 lines of the row group are
// issued before the first is used (LINES = K / 64 for the unrolled widths, 0
// for any other K, which runs in groups of 8 lines). Each 16-byte piece is
// dotted with the matching 8 k of every token, X read from LDS (the lanes of
// one row read consecutive 16 bytes, the lanes of one piece the same ones), as
// four dot2 instructions (two 16-bit products added to an fp32 sum). The 8
// lanes of a row are summed by two quad permutes and a half-row mirror, after
// which lane p holds the row's output for token p. MP: token rows padded to a
// power of two (X rows past M are zeros in LDS and never stored).
template <typename T> struct SkDot;
template <> struct SkDot<bf16_t> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline float dot8(v8 w, v8 x, float acc) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(w, w, 0, 1), __builtin_shufflevector(x, x, 0, 1), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(w, w, 2, 3), __builtin_shufflevector(x, x, 2, 3), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(w, w, 4, 5), __builtin_shufflevector(x, x, 4, 5), acc, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(w, w, 6, 7), __builtin_shufflevector(x, x, 6, 7), acc, false);
  }
};
template <> struct SkDot<f16_t> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  __device__ static inline float dot8(v8 w, v8 x, float acc) {
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(w, w, 0, 1), __builtin_shufflevector(x, x, 0, 1), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(w, w, 2, 3), __builtin_shufflevector(x, x, 2, 3), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_shufflevector(w, w, 4, 5), __builtin_shufflevector(x, x, 4, 5), acc, false);
    return __builtin_amdgcn_fdot2(__builtin_shufflevector(w, w, 6, 7), __builtin_shufflevector(x, x, 6, 7), acc, false);
  }
};

constexpr int kWideThreads = 256;
constexpr int kWideMaxRows = 8;
constexpr int64_t kWideMinGroups = 4096;  // 8-row groups (both weights) for the wide mode
constexpr int kWideGenericLines = 8;

template <typename T, int MP, int LINES>
__global__ __launch_bounds__(kWideThreads) void skinny_wide_kernel(SkArgs a) {
  using D = SkDot<T>;
  using V8 = typename D::v8;
  constexpr int WPB = kWideThreads / 64;
  extern __shared__ __align__(16) unsigned char sk_lds[];
  const int K = a.K;
  const int M = a.M;
  {
    // X -> LDS as MP rows of K elements, rows past M zero.
    const int per_row = K / 8;
    for (int i = threadIdx.x; i < MP * per_row; i += kWideThreads) {
      sku32x4 v = {0u, 0u, 0u, 0u};
      if (i / per_row < M) v = ((const sku32x4*)a.x)[i];
      ((sku32x4*)sk_lds)[i] = v;
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int r = lane >> 3;  // row of the wave's group
  const int p = lane & 7;   // 16-byte piece of each line
  const unsigned char* xp = sk_lds + p * 16;
  for (int64_t g = (int64_t)blockIdx.x * WPB + (threadIdx.x >> 6); g < a.groups;
       g += (int64_t)gridDim.x * WPB) {
    const int which = g >= a.groups0 ? 1 : 0;
    const int64_t N = a.n[which];
    const int64_t n = (g - (which ? a.groups0 : 0)) * 8 + r;
    const sku32x4* wp = (const sku32x4*)((const T*)a.w[which] + (n < N ? n : N - 1) * (int64_t)K) + p;
    float acc[MP];
#pragma unroll
    for (int m = 0; m < MP; ++m) acc[m] = 0.f;
    auto consume = [&](const sku32x4& w, int line) {
      const V8 wv = __builtin_bit_cast(V8, w);
#pragma unroll
      for (int m = 0; m < MP; ++m)
        acc[m] = D::dot8(wv, *(const V8*)(xp + ((int64_t)m * K + line * 64) * 2), acc[m]);
    };
    // Scheduling barriers keep every load ahead of the products and the products
    // line by line: left free, the compiler reads X for all lines before the
    // first product and runs out of registers.
    if constexpr (LINES > 0) {
      sku32x4 w[LINES];
#pragma unroll
      for (int i = 0; i < LINES; ++i) w[i] = __builtin_nontemporal_load(wp + i * 8);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < LINES; ++i) {
        consume(w[i], i);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      const int lines = K / 64;
      for (int c0 = 0; c0 < lines; c0 += kWideGenericLines) {
        sku32x4 w[kWideGenericLines];
#pragma unroll
        for (int i = 0; i < kWideGenericLines; ++i)
          if (c0 + i < lines) w[i] = __builtin_nontemporal_load(wp + (c0 + i) * 8);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < kWideGenericLines; ++i) {
          if (c0 + i < lines) consume(w[i], c0 + i);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    float mine = 0.f;
#pragma unroll
    for (int m = 0; m < MP; ++m) {
      float v = acc[m];
      v += lane_xor1(v);
      v += lane_xor2(v);
      v += dpp_mov<0x141>(v);  // row_half_mirror: the other quad of the row's 8 lanes
      if (p == m) mine = v;
    }
    if (p < M && n < N) {
      const T* bp = (const T*)a.bias[which];
      const float bv = bp ? io<T>::to_f32(bp[n]) : 0.f;
      ((T*)a.y[which])[(int64_t)p * N + n] = io<T>::from_f32(mine + bv);
    }
  }
}

// The grid is sized to the workgroups that are resident at once, since the
// grid-stride loop gives every workgroup an equal share: per CU, the smaller of
// what the kernel's registers allow (looked up once per instantiation) and what
// its LDS (X, MP x K 16-bit elements, of the CU's 160 KiB) allows.
constexpr int64_t kCULds = 160 << 10;

template <typename T, int MP, int LINES>
int skinny_wide_launch(const SkArgs& a, hipStream_t s) {
  static std::atomic<int> by_regs{0};
  const size_t lds = (size_t)MP * a.K * 2;
  int n = by_regs.load(std::memory_order_relaxed);
  if (n == 0) {
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &n, skinny_wide_kernel<T, MP, LINES>, kWideThreads, 0);
    if (e != hipSuccess) return (int)e;
    if (n < 1) n = 1;
    by_regs.store(n, std::memory_order_relaxed);
  }
  const int64_t by_lds = kCULds / (int64_t)lds;
  const int64_t per_cu = by_lds < n ? (by_lds < 1 ? 1 : by_lds) : n;
  const int64_t needed = (a.groups + kWideThreads / 64 - 1) / (kWideThreads / 64);
  const int64_t cap = (int64_t)kSkCUs * per_cu;
  const int64_t blocks = needed < cap ? needed : cap;
  skinny_wide_kernel<T, MP, LINES><<<dim3((unsigned)blocks), dim3(kWideThreads), lds, s>>>(a);
  return launch_status();
}

template <typename T, int MP>
int skinny_wide_lines(const SkArgs& a, hipStream_t s) {
  switch (a.K / 64) {
    case 16: return skinny_wide_launch<T, MP, 16>(a, s);
    case 24: return skinny_wide_launch<T, MP, 24>(a, s);
    case 32: return skinny_wide_launch<T, MP, 32>(a, s);
    default: return skinny_wide_launch<T, MP, 0>(a, s);
  }
}

template <typename T, int SPLIT>
int skinny_launch_split(const SkArgs& a, hipStream_t s) {
  constexpr int NT = SPLIT == 1 ? kSkThreads : 64 * SPLIT;
  constexpr int TPB = SPLIT == 1 ? kSkWaves : 1;
  const int64_t lds = a.M * sk_lds_row(a.K) * 2 + (SPLIT > 1 ? SPLIT * 64 * 4 * 4 : 0);
  const int64_t blocks_needed = (a.tiles + TPB - 1) / TPB;
  const int64_t cap = (int64_t)kSkCUs * kSkBlocksPerCU;
  const int64_t blocks = blocks_needed < cap ? blocks_needed : cap;
  skinny_nt_kernel<T, SPLIT><<<dim3((unsigned)blocks), dim3(NT), (size_t)lds, s>>>(a);
  return launch_status();
}

// Waves per tile: one while the tiles alone give the chip enough waves
// (kSkFillWaves); otherwise 4, 8 or 16 waves share each tile's K, as long as
// each keeps at least kSkMinSteps K steps and X plus the partial tiles (1 KB
// per wave) fit the workgroup's 64 KB of LDS.
constexpr int64_t kSkFillWaves = 2048;
constexpr int kSkMinSteps = 4;

template <typename T>
int skinny_launch(const SkArgs& a, hipStream_t s) {
  const int mp = a.M <= 1 ? 1 : a.M <= 2 ? 2 : a.M <= 4 ? 4 : 8;
  if (a.M <= kWideMaxRows && a.K % 64 == 0 && a.groups >= kWideMinGroups &&
      (int64_t)mp * a.K * 2 <= kSkMaxLds) {
    switch (mp) {
      case 1: return skinny_wide_lines<T, 1>(a, s);
      case 2: return skinny_wide_lines<T, 2>(a, s);
      case 4: return skinny_wide_lines<T, 4>(a, s);
      default: return skinny_wide_lines<T, 8>(a, s);
    }
  }
  if (a.tiles >= kSkFillWaves) return skinny_launch_split<T, 1>(a, s);
  const int steps = a.K / kSkStep;
  const int64_t xlds = a.M * sk_lds_row(a.K) * 2;
  // The smallest split that gives the chip kSkFillWaves waves, or the largest
  // the constraints allow.
  int split = 1;
  for (int cand : {4, 8, 16}) {
    if (steps < cand * kSkMinSteps || xlds + cand * 64 * 4 * 4 > kSkMaxLds) break;
    split = cand;
    if (a.tiles * cand >= kSkFillWaves) break;
  }
  switch (split) {
    case 16: return skinny_launch_split<T, 16>(a, s);
    case 8: return skinny_launch_split<T, 8>(a, s);
    case 4: return skinny_launch_split<T, 4>(a, s);
    default: return skinny_launch_split<T, 1>(a, s);
  }
}

}  // namespace
}  // namespace mqc

using namespace mqc;

extern "C" int mqc_gemm_skinny_nt(const void* X, int64_t M, int64_t K, const void* W1,
                                  const void* bias1, void* Y1, int64_t N1, const void* W2,
                                  const void* bias2, void* Y2, int64_t N2, int dtype,
                                  void* stream) {
  if (M < 0 || K < 0 || N1 < 0 || N2 < 0) return MQC_E_SHAPE;
  if (dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  // K == 0 (an empty reduction) is left to the caller.
  if (M > kSkMaxRows || K == 0 || K % kSkStep != 0) return MQC_E_LIMIT;
  if (M * sk_lds_row(K) * 2 > kSkMaxLds || K >= ((int64_t)1 << 30)) return MQC_E_LIMIT;
  const bool pair = N2 > 0;
  if (M == 0 || (N1 == 0 && !pair)) return MQC_OK;
  if (!X || (N1 > 0 && (!W1 || !Y1)) || (pair && (!W2 || !Y2))) return MQC_E_NULL;
  if (!aligned(X, 16) || (N1 > 0 && (!aligned(W1, 16) || !aligned(Y1, 2))) ||
      (pair && (!aligned(W2, 16) || !aligned(Y2, 2))) || !aligned(bias1, 2) ||
      !aligned(bias2, 2))
    return MQC_E_ALIGN;
  SkArgs a{};
  a.x = X;
  a.w[0] = W1; a.bias[0] = bias1; a.y[0] = Y1; a.n[0] = N1;
  a.w[1] = pair ? W2 : W1; a.bias[1] = pair ? bias2 : bias1;
  a.y[1] = pair ? Y2 : Y1; a.n[1] = pair ? N2 : N1;
  a.tiles0 = (N1 + 15) / 16;
  a.tiles = a.tiles0 + (pair ? (N2 + 15) / 16 : 0);
  a.groups0 = (N1 + 7) / 8;
  a.groups = a.groups0 + (pair ? (N2 + 7) / 8 : 0);
  a.M = (int)M;
  a.K = (int)K;
  if (dtype == MQC_BF16) return skinny_launch<bf16_t>(a, (hipStream_t)stream);
  return skinny_launch<f16_t>(a, (hipStream_t)stream);
}
