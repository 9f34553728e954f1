// The block's B/C projections fused with its SSM walk (bf16 or fp16 storage, fp32
// accumulation): B and C are computed tile by tile in LDS and walked there, so they never
// reach HBM.
//
//   B = x . W_B^T, C = x . W_C^T     (F.linear, mambaqc/layers/quaternion_linear.py:145-161,
//                                     called at models/quaternion_mamba2_block.py:186-191),
//   then the delta/Lambda SSM of ssm_scan.hpp (MODE_DL) on them:
//   h_t = Cayley(delta_t Lambda) (x) h_{t-1} + s_t B_t,  y_t = sum_k C_{t,k} (x) h_{t,k} + D s_t
//                                    (models/quaternion_mamba2_block.py:206-228,
//                                     kernels/ssm_fused.py:363-379,405-430).
//
// Unfused, the two projections write [batch, T, d_inner, d_state, 4] each (12.9 GB in bf16
// at batch 4, T 2048, d_inner 1536, d_state 64) and the walk reads them straight back.
//
// Work decomposition. One workgroup (8 waves) per (b, d), in launch order by d with the
// batches of a d adjacent and each XCD given a contiguous range of d's, so the four
// workgroups that share a d's weight rows and the d's that share a batch's x tile run on
// one L2. The workgroup walks T in tiles of 256 tokens; per tile and per half of the
// states (32 states: 128 rows of W_B and the same 128 rows of W_C):
//   1. GEMM: the 256 x 256 MFMA tile of mfma_tile.hpp, x[b, t0 : t0 + 256, :] against the
//      half's 256 weight rows (B's 128, then C's 128), K = d_inner;
//   2. the tile rounded to the storage dtype (what the projections store, so the walk
//      sees the values the unfused path stores) into LDS over the GEMM's stages, as one 16-byte
//      cell (B quaternion, C quaternion) per (token, state);
//   3. the walk over the tile's 256 tokens for the half's 32 states, by all 8 waves: the
//      tokens in 16 chunks of 16, lane (state k, chunk c);
//        a. each chunk from zero: its transition (P, H), P the product of its q's (in the
//           plane of the state's Lambda_vec: two floats), H its end state;
//        b. a scan over the 16 chunks of each state (one 16-lane row, DPP row shifts, the
//           later transition on the left), the state carried from the previous tile
//           folded into chunk 0: every chunk's start state;
//        c. each chunk again from its start state, with y's terms C (x) h, summed over the
//           32 states by a reduce-scatter across the lanes of a half-wave, into an fp32
//           LDS accumulator of the tile's y (summed over the halves);
//   4. after the last half: y = accumulator + D s, rounded to the storage dtype.
// The state of each half is carried from tile to tile in LDS (fp32), from h0 to h_last.
//
// Split form (a batch of one): one workgroup per (b, d, half), launched d-major with the
// halves adjacent. A d's workgroup streams its weight rows once per tile, and only the
// batches of a d share those reads, so a single sequence's 256 resident d's would want
// 384 MiB of weight rows, more than the Infinity Cache; a half's workgroup wants half of
// that. Each writes its half's fp32 partial sum of the tile's y (step 4 without D s) to
// the caller's workspace, and fused_bc_combine_kernel adds the halves and D s.
#include <atomic>

#include "mfma_tile.hpp"
#include "ssm_chunk.hpp"

namespace mqc {
namespace {

using namespace mfma;

constexpr int kHalf = 32;                 // states per half
constexpr int kMaxHalves = 2;             // d_state <= 64
constexpr int kNChunk = 16;               // chunks per tile
constexpr int kChunkLen = kT / kNChunk;   // 16 tokens
constexpr int kCellBytes = 8;             // one 16-bit quaternion of one (token, state)
constexpr int kTokBytes = kHalf * kCellBytes;  // 256 bytes per token in the B or the C tile
constexpr int kOffC = kT * kTokBytes;          // the C tile after the B tile (64 KiB each)
// LDS layout (bytes): the GEMM's two stages, reused for the B/C tile, then the walk's own.
constexpr int kOffH = kStagesBytes;                          // chunk states [16][32] quat
constexpr int kOffP = kOffH + kNChunk * kHalf * 16;          // chunk products [16][32] float2
constexpr int kOffY = kOffP + kNChunk * kHalf * 8;           // y accumulator [256] float4
constexpr int kOffDS = kOffY + kT * 16;                      // (delta, s) [256] float2
constexpr int kOffHC = kOffDS + kT * 8;                      // carried states [64] quat
constexpr int kOffLT = kOffHC + kMaxHalves * kHalf * 16;     // Cayley constants [64] 2 x float4
constexpr int kLdsFused = kOffLT + kMaxHalves * kHalf * 32;  // 149 KiB

// The B tile is LDS stage 0 and the C tile stage 1: the walk's first pass reads only B,
// the second only C.
static_assert(2 * kT * kTokBytes == kStagesBytes && kOffC == kStageBytes,
              "the B and C tiles are the GEMM's two stages");
static_assert(kLdsFused <= 160 * 1024, "gfx950 LDS");

// 16-bit tensors (bf16 or fp16, the kernel's T) as raw element bits.
struct FusedArgs {
  const uint16_t* x;   // [batch, T, K] (K = d_inner)
  const uint16_t* wb;  // [d_inner * S * 4, K]
  const uint16_t* wc;
  const uint16_t* delta;  // [batch, T, d_inner]
  const uint16_t* s;
  const float* lam_alpha;  // [d_inner, S]
  const float* lam_imag;   // [d_inner, S, 3]
  const float* dvec;       // [d_inner]
  const float* h0;         // [batch, d_inner, S, 4] or null
  uint16_t* y;             // [batch, T, d_inner, 4]
  float* h_last;           // [batch, d_inner, S, 4] or null
  float* ypart;            // split: y's partial sums [halves, batch, T, d_inner, 4]
  int batch, T, Dm, S;
  int split;               // one workgroup per (b, d, half) instead of per (b, d)
  float eps;
};

// The B and C tiles: token t's 32 quaternions (state k at cell k ^ (t & 15)) form one
// 256-byte row, so the 16 tokens one epilogue store instruction writes spread over the
// banks, while the 32 states one walk read takes stay one contiguous row.

// Rows of one K stage for the GEMM tile of (time tile, half): W rows [0, 128) from
// W_B and [128, 256) from W_C, the half's 4 hs rows each (rows past them read the
// half's first state: in a ragged last half the 8-row groups of a DMA instruction are
// whole pairs of states, d_state being even); X rows the tile's tv tokens (rows past
// the sequence read its last token).
struct WRows {
  const uint16_t* wb;
  const uint16_t* wc;
  int64_t row0;
  int hs4, K;
  __device__ const void* operator()(int g, int k0, int i, uint32_t& voff,
                                    const DmaLane& dl) const {
    voff = (uint32_t)(dl.lrow * K * 2) + dl.cb(i);
    const int r = g & 127;  // 8-row groups never straddle B and C
    const int rr = r < hs4 ? r : 0;
    return (g < 128 ? wb : wc) + ((row0 + rr) * K + k0);
  }
};
template <bool FULL_T>
struct XRows {
  const uint16_t* x;
  int64_t row0;
  int tv, K;
  __device__ const void* operator()(int g, int k0, int i, uint32_t& voff,
                                    const DmaLane& dl) const {
    if (FULL_T || tv == kT) {
      voff = (uint32_t)(dl.lrow * K * 2) + dl.cb(i);
      return x + ((row0 + g) * K + k0);
    }
    const int gb = g < tv ? g : tv - 1;
    const int r = g + dl.lrow < tv ? g + dl.lrow : tv - 1;
    voff = (uint32_t)((r - gb) * K * 2) + dl.cb(i);
    return x + ((row0 + gb) * K + k0);
  }
};

// The walk's and the epilogue's LDS addresses are the same for every tile; left to
// itself the compiler computes them once and holds them (tens of registers) through
// the K loop, which then spills. Passing a lane's base through this empty statement
// makes it opaque, so the addresses derived from it are recomputed where used.
template <typename V>
__device__ inline V opaque(V v) {
  asm volatile("" : "+v"(v));
  return v;
}

// The two 16-bit elements of a 32-bit word (low half first) in fp32.
template <typename T>
__device__ inline float lo16(uint32_t w) {
  if constexpr (std::is_same<T, bf16_t>::value) return __uint_as_float(w << 16);
  else return io<T>::bits_to_f32(w & 0xffffu);
}
template <typename T>
__device__ inline float hi16(uint32_t w) {
  if constexpr (std::is_same<T, bf16_t>::value) return __uint_as_float(w & 0xffff0000u);
  else return io<T>::bits_to_f32(w >> 16);
}

// Exchange x of the odd 16-lane rows with y of the even rows (v_permlane16_swap_b32):
// afterwards even-row lanes hold (own x, the odd neighbour's x) and odd-row lanes
// (the even neighbour's y, own y). Issued as assembly with both registers read-write,
// as the library's other row swaps (common.hpp), N pairs behind one pair of s_nops.
template <int N>
__device__ inline void row_swap16(float* x, float* y) {
  static_assert(N == 8, "eight pairs per statement");
  asm volatile(
      "s_nop 1\n\t"
      "v_permlane16_swap_b32 %0, %8\n\t"
      "v_permlane16_swap_b32 %1, %9\n\t"
      "v_permlane16_swap_b32 %2, %10\n\t"
      "v_permlane16_swap_b32 %3, %11\n\t"
      "v_permlane16_swap_b32 %4, %12\n\t"
      "v_permlane16_swap_b32 %5, %13\n\t"
      "v_permlane16_swap_b32 %6, %14\n\t"
      "v_permlane16_swap_b32 %7, %15\n\t"
      "s_nop 1"
      : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]),
        "+v"(x[7]), "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]), "+v"(y[4]), "+v"(y[5]),
        "+v"(y[6]), "+v"(y[7]));
}

__device__ inline float row_half_mirror(float v) { return dpp_mov<0x141>(v); }

// Sum of o[64] (16 tokens x 4 components of one chunk, i = 4 j + comp) over the 32 lanes
// of each half-wave, scattered: lane u (= lane & 31) ends with the sums of indices
// i0 = 32 * (1 - u4) + 2 * (u & 15) and i0 + 1 (u4 = bit 4 of u). Butterfly stages at
// lane distances 16 (row swap), 8 (row rotation), 4 (half-row mirror: pairs lanes
// p and 7 - p of each 8), 2 and 1 (quad permutes); at each stage a lane keeps half of its
// values and adds its partner's copies of them.
__device__ inline void reduce_scatter32(float (&o)[64], int lane, float& r0, float& r1) {
  float w[32];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    float xs[8], ys[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      xs[i] = o[32 + 8 * g + i];
      ys[i] = o[8 * g + i];
    }
    row_swap16<8>(xs, ys);
    // Even rows: own o[32 + i] + neighbour's o[32 + i]; odd rows: neighbour's o[i] + own o[i].
#pragma unroll
    for (int i = 0; i < 8; ++i) w[8 * g + i] = xs[i] + ys[i];
  }
  const bool b3 = lane & 8, b2 = lane & 4, b1 = lane & 2, b0 = lane & 1;
  float z[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float send = b3 ? w[i] : w[16 + i];
    const float keep = b3 ? w[16 + i] : w[i];
    z[i] = keep + row_rot8(send);
  }
  float r8[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float send = b2 ? z[i] : z[8 + i];
    const float keep = b2 ? z[8 + i] : z[i];
    r8[i] = keep + row_half_mirror(send);
  }
  float r4[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float send = b1 ? r8[i] : r8[4 + i];
    const float keep = b1 ? r8[4 + i] : r8[i];
    r4[i] = keep + lane_xor2(send);
  }
  float r2[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float send = b0 ? r4[i] : r4[2 + i];
    const float keep = b0 ? r4[2 + i] : r4[i];
    r2[i] = keep + lane_xor1(send);
  }
  r0 = r2[0];
  r1 = r2[1];
}

// T: the 16-bit storage type (bf16_t or f16_t), whose MFMAs the GEMM runs. FULL_T: the
// sequence length is a multiple of 256 (no ragged last tile). FULL_S: d_state is a
// multiple of 32 (every half full).
template <typename T, bool FULL_T, bool FULL_S>
__global__ __launch_bounds__(kThreads) void fused_bc_ssm_kernel(FusedArgs a) {
  using E = typename std::conditional<std::is_same<T, bf16_t>::value, __bf16, _Float16>::type;
  extern __shared__ __attribute__((aligned(1024))) char lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave >> 2;
  const int wm = wave & 3;
  const int rl = lane & 15;
  const int q4 = lane >> 4;

  // Unit (b, d), or (b, d, half) when split: logical order d-major (then the half)
  // with the batches adjacent, each XCD a contiguous range of it (blocks go to the
  // XCDs round-robin by linear id).
  const int n = (int)gridDim.x;
  const int lin = (int)blockIdx.x;
  const int logical = n % kXCDs ? lin : (lin % kXCDs) * (n / kXCDs) + lin / kXCDs;
  const int K = a.Dm;
  const int S = a.S;
  const int NH = (S + kHalf - 1) / kHalf;
  const int per_d = a.split ? a.batch * NH : a.batch;
  const int d = __builtin_amdgcn_readfirstlane(logical / per_d);
  const int rem = logical - d * per_d;
  const int hsel = __builtin_amdgcn_readfirstlane(a.split ? rem / a.batch : 0);
  const int b = __builtin_amdgcn_readfirstlane(rem - hsel * a.batch);
  const int h_begin = a.split ? hsel : 0;
  const int h_end = a.split ? hsel + 1 : NH;
  const int64_t bd = (int64_t)b * a.Dm + d;

  // Walk mapping A: state kA of the half, chunk cA (tokens cA * 16 + [0, 16)).
  const int kA = lane & 31;
  const int cA = wave * 2 + (lane >> 5);
  // Scan mapping: state kS, chunk cS; the 16 chunks of a state are one 16-lane row.
  const int kS = tid >> 4;
  const int cS = tid & 15;

  // Per-state constants of the Cayley closed form in an LDS table, (v, |v|^2) and
  // (a, n2, -, -) per state (kept out of registers, which the K loop fills); states past
  // S are clamped onto S - 1 and their results discarded.
  if (tid < kMaxHalves * kHalf) {
    const int k = tid < S ? tid : S - 1;
    const LamConst L = lam_const(a.lam_alpha, a.lam_imag, (int64_t)d * S + k);
    const float4 lv = {L.v0, L.v1, L.v2, L.v0 * L.v0 + L.v1 * L.v1 + L.v2 * L.v2};
    const float4 la = {L.a, L.n2, 0.f, 0.f};
    *(float4*)(lds + kOffLT + tid * 32) = lv;
    *(float4*)(lds + kOffLT + tid * 32 + 16) = la;
    float4 hc = {0.f, 0.f, 0.f, 0.f};
    if (a.h0 && tid < S) hc = *(const float4*)(a.h0 + (bd * S + tid) * 4);
    *(float4*)(lds + kOffHC + tid * 16) = hc;
  }

  const int n_tiles = (a.T + kT - 1) / kT;
  auto wrows = [&](int h) {
    const int hs = FULL_S ? kHalf : (S - h * kHalf < kHalf ? S - h * kHalf : kHalf);
    return WRows{a.wb, a.wc, ((int64_t)d * S + h * kHalf) * 4, 4 * hs, K};
  };
  auto xrows = [&](int ti) {
    const int tv = FULL_T ? kT : (a.T - ti * kT < kT ? a.T - ti * kT : kT);
    return XRows<FULL_T>{a.x, (int64_t)b * a.T + ti * kT, tv, K};
  };
  // delta and s of time tile ti, one token per thread of the first 256 (zero past the
  // sequence: no input; the walk takes q = 1 there, so padded steps leave the state as
  // it is). Held in registers until the tile's first K loop has waited for them, then
  // stored to LDS.
  float dl_t = 0.f, s_t = 0.f;
  auto load_ds = [&](int ti) {
    const int tv = FULL_T ? kT : (a.T - ti * kT < kT ? a.T - ti * kT : kT);
    dl_t = 0.f;
    s_t = 0.f;
    if (tid < kT && tid < tv) {
      const int64_t e = ((int64_t)b * a.T + ti * kT + tid) * a.Dm + d;
      dl_t = io<T>::bits_to_f32(a.delta[e]);
      s_t = io<T>::bits_to_f32(a.s[e]);
    }
  };
  if (n_tiles > 0) load_ds(0);
  for (int ti = 0; ti < n_tiles; ++ti) {
    const int tv = FULL_T ? kT : (a.T - ti * kT < kT ? a.T - ti * kT : kT);
    const int64_t xrow0 = (int64_t)b * a.T + ti * kT;
    for (int h = h_begin; h < h_end; ++h) {
      // ---- 1. GEMM tile: rows [0, 128) of W_B, then [0, 128) of W_C, for the half's
      // states, against the tile's tokens.
      const int hs = FULL_S ? kHalf : (S - h * kHalf < kHalf ? S - h * kHalf : kHalf);  // states in this half
      floatx4 acc[kWB][kXB];
#pragma unroll
      for (int i = 0; i < kWB; ++i)
#pragma unroll
        for (int j = 0; j < kXB; ++j) acc[i][j] = (floatx4){};
      tile_kloop<E>(K, lds, acc, wrows(h), xrows(ti));
      if (h == h_begin && tid < kT) *(float2*)(lds + kOffDS + tid * 8) = float2{dl_t, s_t};

      // ---- 2. The tile, rounded to T, over the stages (every wave is past its last
      // fragment read at the barrier).
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();
      {
        // Cell of (t = wm * 64 + mb * 16 + rl, k = nb * 4 + q4) in the B (wn = 0) or C
        // (wn = 1) tile: k ^ (t & 15) = (nb * 4) ^ (q4 ^ rl), a constant per block XORed
        // with the lane's x0.
        const uint32_t base = opaque((uint32_t)(wn * kOffC + (wm * 64 + rl) * kTokBytes));
        const uint32_t x0 = opaque((uint32_t)(q4 ^ rl));
#pragma unroll
        for (int nb = 0; nb < kWB; ++nb)
#pragma unroll
          for (int mb = 0; mb < kXB; ++mb) {
            const uint32_t cst = (uint32_t)(nb * 4);
            const floatx4& v = acc[nb][mb];
            const u32x2 pk = {pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])};
            *(u32x2*)(lds + base + mb * 16 * kTokBytes + ((x0 ^ cst) << 3)) = pk;
          }
      }
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();

      // ---- 3a. Every chunk from zero: its local states hl_j and the prefix products
      // P_j = q_j ... q_0 (kept in registers for 3c), and its transition (P_15, hl_15).
      LamConst L;
      float vv;
      {
        const float4 lv = *(const float4*)(lds + kOffLT + (h * kHalf + kA) * 32);
        const float4 la = *(const float4*)(lds + kOffLT + (h * kHalf + kA) * 32 + 16);
        L.v0 = lv.x;
        L.v1 = lv.y;
        L.v2 = lv.z;
        vv = lv.w;
        L.a = la.x;
        L.n2 = la.y;
      }
      quat hl[kChunkLen];
      float pa[kChunkLen], pb[kChunkLen];
      {
        quat hh{0.f, 0.f, 0.f, 0.f};
        float ca = 1.f, cb = 0.f;
        // Token t = cA * 16 + j: t & 15 = j, so state k's cell is k ^ j.
        const uint32_t tb = opaque((uint32_t)(cA * kChunkLen));
        const uint32_t kx = opaque((uint32_t)kA);
#pragma unroll
        for (int j = 0; j < kChunkLen; ++j) {
          const uint32_t t = tb + j;
          const float2 ds = *(const float2*)(lds + kOffDS + t * 8);
          const u32x2 br = *(const u32x2*)(lds + t * kTokBytes + ((kx ^ j) << 3));
          const quat Bq{lo16<T>(br[0]), hi16<T>(br[0]), lo16<T>(br[1]), hi16<T>(br[1])};
          float c;
          quat qq = cayley_step_c(ds.x, ds.x * ds.x, L, a.eps, c);
          if constexpr (!FULL_T) {
            // Past the sequence q is the identity, not Cayley(0) = 1 / max(1, eps).
            if ((int)t >= tv) {
              qq = quat{1.f, 0.f, 0.f, 0.f};
              c = 0.f;
            }
          }
          hh = state_step(qq, hh, ds.y, Bq);
          const float na = fmaf(qq.w, ca, -c * cb * vv);
          cb = fmaf(qq.w, cb, c * ca);
          ca = na;
          hl[j] = hh;
          pa[j] = ca;
          pb[j] = cb;
        }
        *(float4*)(lds + kOffH + (cA * kHalf + kA) * 16) = float4{hh.w, hh.x, hh.y, hh.z};
        *(float2*)(lds + kOffP + (cA * kHalf + kA) * 8) = float2{ca, cb};
      }
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();
      // The next time tile's delta and s, loaded during the scan and the second pass.
      // (Loading the next GEMM tile's first K stage into the B tile here, LDS stage 0,
      // which the walk has read by now, measured no faster: 16.48-16.61 against
      // 16.45-16.46 ms at config 3, same box.)
      if (h + 1 == h_end && ti + 1 < n_tiles) load_ds(ti + 1);

      // ---- 3b. Start states: an inclusive scan over each state's 16 chunks (row shifts
      // of 1, 2, 4, 8 within the 16-lane row), the carried state folded into chunk 0.
      {
        const float4 e = *(const float4*)(lds + kOffH + (cS * kHalf + kS) * 16);
        const float2 p = *(const float2*)(lds + kOffP + (cS * kHalf + kS) * 8);
        const float4 lt = *(const float4*)(lds + kOffLT + (h * kHalf + kS) * 32);
        const float4 hc = *(const float4*)(lds + kOffHC + (h * kHalf + kS) * 16);
        LamConst LS{};
        LS.v0 = lt.x;
        LS.v1 = lt.y;
        LS.v2 = lt.z;
        const float vvS = lt.w;
        const quat carry{hc.x, hc.y, hc.z, hc.w};
        ChunkMap m;
        m.pa = p.x;
        m.pb = p.y;
        m.H = quat{e.x, e.y, e.z, e.w};
        if (cS == 0) {
          const quat ph = vplane_mul(m.pa, m.pb, LS, carry);
          m.H = quat{ph.w + m.H.w, ph.x + m.H.x, ph.y + m.H.y, ph.z + m.H.z};
        }
        const ChunkMap e1 = dpp_map<0x111, 0xF>(m);  // row_shr:1
        if (cS >= 1) m = compose(m, e1, vvS, LS);
        const ChunkMap e2 = dpp_map<0x112, 0xF>(m);  // row_shr:2
        if (cS >= 2) m = compose(m, e2, vvS, LS);
        const ChunkMap e4 = dpp_map<0x114, 0xF>(m);  // row_shr:4
        if (cS >= 4) m = compose(m, e4, vvS, LS);
        const ChunkMap e8 = dpp_map<0x118, 0xF>(m);  // row_shr:8
        if (cS >= 8) m = compose(m, e8, vvS, LS);
        // m.H: the state at the end of chunk cS = the start of chunk cS + 1. Each
        // state's 16 chunks are one row of one wave, whose reads above all precede
        // these writes.
        const float4 mh = {m.H.w, m.H.x, m.H.y, m.H.z};
        if (cS < kNChunk - 1)
          *(float4*)(lds + kOffH + ((cS + 1) * kHalf + kS) * 16) = mh;
        else if (h * kHalf + kS < S)
          *(float4*)(lds + kOffHC + (h * kHalf + kS) * 16) = mh;
        if (cS == 0) *(float4*)(lds + kOffH + kS * 16) = hc;
      }
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();

      // ---- 3c. Every chunk's states from its start state h_s:
      //   h_j = P_j (x) h_s + hl_j = pa_j h_s + pb_j (v (x) h_s) + hl_j,
      // and y's terms C_j (x) h_j.
      {
        const float4 e = *(const float4*)(lds + kOffH + (cA * kHalf + kA) * 16);
        const quat hs0{e.x, e.y, e.z, e.w};
        const quat vh = qmul(quat{0.f, L.v0, L.v1, L.v2}, hs0);
        float o[4 * kChunkLen];
        const bool live = FULL_S || kA < hs;
        const uint32_t tb = opaque((uint32_t)(cA * kChunkLen));
        const uint32_t kx = opaque((uint32_t)kA);
#pragma unroll
        for (int j = 0; j < kChunkLen; ++j) {
          const uint32_t t = tb + j;
          const u32x2 r = *(const u32x2*)(lds + kOffC + t * kTokBytes + ((kx ^ j) << 3));
          const quat Cq{lo16<T>(r[0]), hi16<T>(r[0]), lo16<T>(r[1]), hi16<T>(r[1])};
          const quat hh{fmaf(pa[j], hs0.w, fmaf(pb[j], vh.w, hl[j].w)),
                        fmaf(pa[j], hs0.x, fmaf(pb[j], vh.x, hl[j].x)),
                        fmaf(pa[j], hs0.y, fmaf(pb[j], vh.y, hl[j].y)),
                        fmaf(pa[j], hs0.z, fmaf(pb[j], vh.z, hl[j].z))};
          const quat oc = qmul(Cq, hh);
          o[4 * j + 0] = live ? oc.w : 0.f;
          o[4 * j + 1] = live ? oc.x : 0.f;
          o[4 * j + 2] = live ? oc.y : 0.f;
          o[4 * j + 3] = live ? oc.z : 0.f;
        }
        float r0, r1;
        reduce_scatter32(o, lane, r0, r1);
        const int u = lane & 31;
        const int i0 = ((u & 16) ? 0 : 32) + 2 * (u & 15);
        const int t = cA * kChunkLen + (i0 >> 2);
        float2* yp = (float2*)(lds + kOffY + t * 16 + (i0 & 3) * 4);
        if (h == h_begin) {
          *yp = float2{r0, r1};
        } else {
          const float2 prev = *yp;
          *yp = float2{prev.x + r0, prev.y + r1};
        }
      }
      // The next K loop refills the stages (the B/C tile) and the next half adds to y.
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();
    }
    // ---- 4. y of the tile, or (split) this half's partial sum of it.
    if (tid < tv) {
      const float4 yv = *(const float4*)(lds + kOffY + tid * 16);
      if (a.split) {
        const int64_t row = (int64_t)hsel * a.batch * a.T + xrow0 + tid;
        *(float4*)(a.ypart + (row * a.Dm + d) * 4) = yv;
      } else {
        const float dsk = a.dvec[d];
        const float sv = (*(const float2*)(lds + kOffDS + tid * 8)).y;
        const u32x2 pk = {pack2<T>(fmaf(dsk, sv, yv.x), yv.y), pack2<T>(yv.z, yv.w)};
        *(u32x2*)(a.y + ((xrow0 + tid) * a.Dm + d) * 4) = pk;
      }
    }
    // (The next tile's first LDS writes of y and of (delta, s) come after barriers.)
  }
  __syncthreads();  // (with no tiles: the carried states' LDS writes above)
  if (a.h_last && tid < S && tid >= h_begin * kHalf && tid < h_end * kHalf) {
    const float4 hc = *(const float4*)(lds + kOffHC + tid * 16);
    *(float4*)(a.h_last + (bd * S + tid) * 4) = hc;
  }
}

// The split walk's second launch: y = T(p0 + p1 + (D s, 0, 0, 0)) per (b, t, d), the
// sum in the order the unsplit kernel makes it (half 0's partial, then half 1's, then
// D s), so both forms give the same y bit for bit.
template <typename T>
__global__ __launch_bounds__(256) void fused_bc_combine_kernel(const float* __restrict__ ypart,
                                                               const uint16_t* __restrict__ s,
                                                               const float* __restrict__ dvec,
                                                               uint16_t* __restrict__ y,
                                                               int64_t n, int64_t half_stride,
                                                               int Dm) {
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n;
       e += (int64_t)gridDim.x * blockDim.x) {
    const float4 p0 = *(const float4*)(ypart + e * 4);
    const float4 p1 = *(const float4*)(ypart + (half_stride + e) * 4);
    const float sv = io<T>::bits_to_f32(s[e]);
    const float dsk = dvec[e % Dm];
    const u32x2 pk = {pack2<T>(fmaf(dsk, sv, p0.x + p1.x), p0.y + p1.y),
                      pack2<T>(p0.z + p1.z, p0.w + p1.w)};
    *(u32x2*)(y + e * 4) = pk;
  }
}

}  // namespace
}  // namespace mqc

using namespace mqc;

namespace {
constexpr int kMaxDevices = 64;
std::atomic<bool> g_fused_attr_set[kMaxDevices];

template <typename K>
int set_lds_limit(K kernel) {
  return (int)hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  kLdsFused);
}

template <typename T>
int set_lds_limits() {
  int st = set_lds_limit(fused_bc_ssm_kernel<T, true, true>);
  if (st == MQC_OK) st = set_lds_limit(fused_bc_ssm_kernel<T, true, false>);
  if (st == MQC_OK) st = set_lds_limit(fused_bc_ssm_kernel<T, false, true>);
  if (st == MQC_OK) st = set_lds_limit(fused_bc_ssm_kernel<T, false, false>);
  return st;
}

template <typename T>
void launch_fused(const FusedArgs& a, dim3 grid, bool full_t, bool full_s, hipStream_t st) {
  if (full_t && full_s)
    hipLaunchKernelGGL((fused_bc_ssm_kernel<T, true, true>), grid, dim3(kThreads), kLdsFused, st, a);
  else if (full_t)
    hipLaunchKernelGGL((fused_bc_ssm_kernel<T, true, false>), grid, dim3(kThreads), kLdsFused, st, a);
  else if (full_s)
    hipLaunchKernelGGL((fused_bc_ssm_kernel<T, false, true>), grid, dim3(kThreads), kLdsFused, st, a);
  else
    hipLaunchKernelGGL((fused_bc_ssm_kernel<T, false, false>), grid, dim3(kThreads), kLdsFused, st, a);
}
}  // namespace

namespace {

int64_t split_workspace_bytes(int64_t batch, int64_t seq_len, int64_t d_inner, int64_t d_state) {
  if (batch <= 0 || seq_len <= 0 || d_inner <= 0 || d_state <= kHalf) return 0;
  return 2 * batch * seq_len * d_inner * 4 * (int64_t)sizeof(float);
}

int fused_bc_run(const void* x, const void* B_weight, const void* C_weight, const void* delta,
                 const void* s, const float* lambda_alpha, const float* lambda_imag,
                 const float* D, const void* h0, void* y, void* h_last, int64_t batch,
                 int64_t seq_len, int64_t d_inner, int64_t d_state, float eps, int dtype,
                 bool split, void* workspace, int64_t workspace_bytes, void* stream) {
  if (batch < 0 || seq_len < 0 || d_inner < 0 || d_state < 0) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  if (dtype == MQC_F32) return MQC_E_DTYPE;  // 16-bit MFMAs only
  if (batch == 0 || d_inner == 0) return MQC_OK;
  if (d_state < 1 || d_state > kMaxHalves * kHalf) return MQC_E_LIMIT;
  if (d_state % 2 != 0) return MQC_E_SHAPE;  // 8-row DMA groups of whole states
  if (d_inner % kBK != 0) return MQC_E_SHAPE;
  if (seq_len > 0 && (!x || !B_weight || !C_weight || !delta || !s || !y)) return MQC_E_NULL;
  if (!lambda_alpha || !lambda_imag || !D) return MQC_E_NULL;
  if (!aligned(x, 16) || !aligned(B_weight, 16) || !aligned(C_weight, 16) || !aligned(y, 8) ||
      !aligned(delta, 2) || !aligned(s, 2) || (h0 && !aligned(h0, 16)) ||
      (h_last && !aligned(h_last, 16)))
    return MQC_E_ALIGN;
  // 32-bit token and unit indices; one (b, d) (or (b, d, half)) per workgroup.
  if (batch * d_inner * kMaxHalves > 0x7fffffffLL || batch * seq_len > (1LL << 30) ||
      d_inner > (1 << 20))
    return MQC_E_LIMIT;
  // Split only where there are two halves and steps to walk; its partial sums go to
  // the workspace.
  split = split && split_workspace_bytes(batch, seq_len, d_inner, d_state) > 0;
  if (split) {
    if (!workspace) return MQC_E_NULL;
    if (!aligned(workspace, 16)) return MQC_E_ALIGN;
    if (workspace_bytes < split_workspace_bytes(batch, seq_len, d_inner, d_state))
      return MQC_E_SPACE;
  }
  // Each (b, d) reads h0 and writes h_last for its own states only, after its walk:
  // h_last may be h0, but not a shifted alias of it.
  if (partial_overlap(h0, h_last, batch * d_inner * d_state * 4 * (int64_t)sizeof(float)))
    return MQC_E_OVERLAP;
  if (seq_len == 0 && !h_last) return MQC_OK;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return MQC_E_LIMIT;
  if (!g_fused_attr_set[dev].load(std::memory_order_acquire)) {
    int st = set_lds_limits<bf16_t>();
    if (st == MQC_OK) st = set_lds_limits<f16_t>();
    if (st != MQC_OK) return st;
    g_fused_attr_set[dev].store(true, std::memory_order_release);
  }
  FusedArgs a{};
  a.x = (const uint16_t*)x; a.wb = (const uint16_t*)B_weight; a.wc = (const uint16_t*)C_weight;
  a.delta = (const uint16_t*)delta; a.s = (const uint16_t*)s;
  a.lam_alpha = lambda_alpha; a.lam_imag = lambda_imag; a.dvec = D;
  a.h0 = (const float*)h0; a.y = (uint16_t*)y; a.h_last = (float*)h_last;
  a.ypart = split ? (float*)workspace : nullptr;
  a.batch = (int)batch; a.T = (int)seq_len; a.Dm = (int)d_inner; a.S = (int)d_state; a.eps = eps;
  a.split = split ? 1 : 0;
  const int64_t units = batch * d_inner * (split ? kMaxHalves : 1);
  const dim3 grid((unsigned)units);
  hipStream_t st = (hipStream_t)stream;
  const bool full_t = seq_len % kT == 0, full_s = d_state % kHalf == 0;
  if (dtype == MQC_BF16)
    launch_fused<bf16_t>(a, grid, full_t, full_s, st);
  else
    launch_fused<f16_t>(a, grid, full_t, full_s, st);
  if (!split) return launch_status();
  int status = launch_status();
  if (status != MQC_OK) return status;
  const int64_t n = batch * seq_len * d_inner;
  const int64_t blocks = (n + 255) / 256 < 16384 ? (n + 255) / 256 : 16384;
  if (dtype == MQC_BF16)
    hipLaunchKernelGGL(fused_bc_combine_kernel<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const float*)workspace, (const uint16_t*)s, D, (uint16_t*)y, n, n,
                       (int)d_inner);
  else
    hipLaunchKernelGGL(fused_bc_combine_kernel<f16_t>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const float*)workspace, (const uint16_t*)s, D, (uint16_t*)y, n, n,
                       (int)d_inner);
  return launch_status();
}

}  // namespace

extern "C" {

int mqc_ssm_fused_bc_fwd(const void* x, const void* B_weight, const void* C_weight,
                         const void* delta, const void* s, const float* lambda_alpha,
                         const float* lambda_imag, const float* D, const void* h0, void* y,
                         void* h_last, int64_t batch, int64_t seq_len, int64_t d_inner,
                         int64_t d_state, float eps, int dtype, void* stream) {
  return fused_bc_run(x, B_weight, C_weight, delta, s, lambda_alpha, lambda_imag, D, h0, y,
                      h_last, batch, seq_len, d_inner, d_state, eps, dtype, false, nullptr, 0,
                      stream);
}

int64_t mqc_ssm_fused_bc_split_workspace_bytes(int64_t batch, int64_t seq_len, int64_t d_inner,
                                               int64_t d_state) {
  if (batch < 0 || seq_len < 0 || d_inner < 0 || d_state < 0) return MQC_E_SHAPE;
  return split_workspace_bytes(batch, seq_len, d_inner, d_state);
}

int mqc_ssm_fused_bc_fwd_split(const void* x, const void* B_weight, const void* C_weight,
                               const void* delta, const void* s, const float* lambda_alpha,
                               const float* lambda_imag, const float* D, const void* h0,
                               void* y, void* h_last, int64_t batch, int64_t seq_len,
                               int64_t d_inner, int64_t d_state, float eps, int dtype,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  return fused_bc_run(x, B_weight, C_weight, delta, s, lambda_alpha, lambda_imag, D, h0, y,
                      h_last, batch, seq_len, d_inner, d_state, eps, dtype, true, workspace,
                      workspace_bytes, stream);
}

}  // extern "C"
