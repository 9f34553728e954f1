#pragma once
// Quaternion selective-state-space recurrence, fused.
//
//   h_t = q_t (x) h_{t-1} + B_t (x) S_t        (S broadcast over d_state)
//   y_t = sum_k C_{t,k} (x) h_{t,k} + D_t * S_t
//
// (mambaqc/kernels/ssm_fused.py:363-379 and :405-430.)
//
// Two operand forms share one kernel:
//   MODE_DL  the block's form: q_t = Cayley(delta_t * Lambda) is computed in
//            registers from a per-(d,k) Lambda (closed form below), S = (s,0,0,0)
//            so B (x) S = s * B, and D is a per-d vector. Neither z nor q is
//            ever written to memory (quaternion_mamba2_block.py:183-228).
//   MODE_Q   q, S (full quaternion) and D (strided [B,T,D]) given explicitly,
//            as in ssm_forward_fused / ssm_step_fused.
//
// Work decomposition. Every (b, d, k) is an independent sequential recurrence
// over t. The grid is (d-blocks, batch), remapped so that each XCD runs a
// contiguous range of blocks (xcd_block: 1 % faster at config 3, neighbouring
// blocks share lines of delta, s and y); the batch row is uniform, so the
// start of every (b, t) slice is a wave-uniform scalar and each lane only
// carries a 32-bit offset inside the slice. A group of G consecutive lanes
// owns one (b, d); lane j of the group owns KPL states (one lane reads
// KPL*4 elements of B and of C per step: 16 bytes for bf16 with KPL = 2,
// contiguous; 32 bytes as two 16-byte pieces half a row apart, see SPLIT in
// the kernel). Lanes past the last d or the last k are clamped onto valid
// addresses instead of being branched around, so the per-step loads carry no
// predicate; their results are discarded (past-d groups store nothing,
// past-k lanes are zeroed before the k-sum).
//
// Each lane walks all T steps with its KPL states in registers and a ring of
// PF steps of operands in flight (raw bits, unpacked when consumed). A slot is
// consumed before it is refilled with step t+PF, so the ring needs no copies.
// The waves of a block are kept on the same step by a barrier (see
// launch_ssm_shape), which keeps each block's reads of a (b, t) slice together.
//
// The per-step sum over k: an FMA chain over the lane's KPL states, then a
// G-lane transpose-reduce on the VALU. The first two butterfly stages (DPP
// quad permutes) swap half of the four components with the partner lane
// instead of reducing all four, so afterwards each lane carries one component
// and the remaining stages are single adds: DPP row rotations by 4 and 8 inside
// a 16-lane row, then permlane16/permlane32 swaps across rows.
//
// Cayley closed form. For z = (a, v), den = 1 - z/2, num = 1 + z/2:
//   den^-1 (x) num = (1 - |z|^2/4, v) / max(|den|^2, eps),
//   |den|^2 = 1 - a + |z|^2/4,
// because conj(den) and num share v's axis and therefore commute. With
// z = delta * Lambda and n2 = |Lambda|^2 / 4 per (d, k):
//   N = max(1 - delta*a_L + delta^2 n2, eps),
//   q = ((1 - delta^2 n2) / N, delta * v_L / N),
// one reciprocal per (t, d, k).
#include <type_traits>

#include "common.hpp"

namespace mqc {

constexpr int MODE_DL = 0;
constexpr int MODE_Q = 1;
constexpr int kSsmThreads = 256;

// Raw bits of N consecutive storage elements (unpacked only on use). A single
// 16-bit element is kept in a 16-bit field: held in 32 bits, the zero-extension
// of a 16-bit buffer load is materialised (v_and) right after the load is
// issued, with a wait for that load in front of it, which stalls the wave on
// every prefetch; in 16 bits it folds into the unpack at the point of use.
template <int BYTES>
struct RawBits {
  uint32_t w[(BYTES + 3) / 4];
  __device__ uint32_t word(int i) const { return w[i]; }
};
template <>
struct RawBits<2> {
  uint16_t h;
  __device__ uint32_t word(int) const { return h; }
};
template <typename T, int N>
struct Raw : RawBits<N * (int)sizeof(T)> {
  static constexpr int W = (N * (int)sizeof(T) + 3) / 4;
};

// Buffer resource over memory from p on: raw (unswizzled), stride 0, the
// maximum record count, gfx9's 32-bit data-format word. Loads through it take
// a scalar base (rebuilt per step from SGPRs) plus a 32-bit per-lane offset in
// one VGPR, so the per-step addressing costs no VALU instructions; with global
// loads the compiler keeps a 64-bit lane pointer per tensor and adds the step
// offset to it on the VALU every step.
__device__ inline __amdgpu_buffer_rsrc_t buf_rsrc(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, -1, 0x00020000);
}

// Load N elements at byte offset voff (per lane) + soff (wave-uniform, added
// by the buffer unit from an SGPR) of a buffer. Loads of 16 bytes or more come
// as 16-byte pieces STRIDE bytes apart (16: contiguous), or a 16-byte load with
// another STRIDE as two 8-byte pieces; AUX is the cache policy of the 16- and
// 8-byte loads (0, or 2 = NT for streams read once).
template <typename T, int N, int AUX = 0, int STRIDE = 16>
__device__ inline void raw_load_buf(__amdgpu_buffer_rsrc_t rs, uint32_t voff, Raw<T, N>& r,
                                    uint32_t soff = 0) {
  constexpr int bytes = N * (int)sizeof(T);
  if constexpr (STRIDE != 16 && bytes == 16) {
    // Two 8-byte pieces STRIDE bytes apart.
    const auto v0 = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, AUX);
    const auto v1 = __builtin_amdgcn_raw_buffer_load_b64(rs, voff + STRIDE, soff, AUX);
    r.w[0] = v0[0]; r.w[1] = v0[1]; r.w[2] = v1[0]; r.w[3] = v1[1];
  } else if constexpr (bytes % 16 == 0) {
#pragma unroll
    for (int i = 0; i < bytes / 16; ++i) {
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + STRIDE * i, soff, AUX);
      r.w[4 * i + 0] = v[0];
      r.w[4 * i + 1] = v[1];
      r.w[4 * i + 2] = v[2];
      r.w[4 * i + 3] = v[3];
    }
  } else if constexpr (bytes == 8) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, AUX);
    r.w[0] = v[0];
    r.w[1] = v[1];
  } else if constexpr (bytes == 4) {
    r.w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, 0);
  } else {
    static_assert(bytes == 2, "unsupported raw width");
    r.h = __builtin_amdgcn_raw_buffer_load_b16(rs, voff, soff, 0);
  }
}

// Store one element (converted from fp32) at byte offset voff + soff of a buffer.
template <typename T>
__device__ inline void store_elem_buf(__amdgpu_buffer_rsrc_t rs, uint32_t voff, float v,
                                      uint32_t soff = 0) {
  if constexpr (sizeof(T) == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rs, voff, soff, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16(io<T>::from_f32(v).bits, rs, voff, soff, 0);
  }
}

template <typename T, int N>
__device__ inline float raw_get(const Raw<T, N>& r, int e) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(r.word(e));
  } else if constexpr (std::is_same<T, bf16_t>::value) {
    const uint32_t word = r.word(e >> 1);
    return __uint_as_float((e & 1) ? (word & 0xffff0000u) : (word << 16));
  } else {
    const uint32_t word = r.word(e >> 1);
    return io<T>::bits_to_f32((e & 1) ? (word >> 16) : (word & 0xffffu));
  }
}

template <typename T, int N>
__device__ inline quat raw_quat(const Raw<T, N>& r, int qi) {
  return quat{raw_get(r, 4 * qi + 0), raw_get(r, 4 * qi + 1), raw_get(r, 4 * qi + 2),
              raw_get(r, 4 * qi + 3)};
}

struct SsmArgs {
  // MODE_DL: delta, s [B,T,D]; lam_alpha [D,S]; lam_imag [D,S,3]; dvec [D]
  const void* delta;
  const void* s;
  const float* lam_alpha;
  const float* lam_imag;
  const float* dvec;
  // MODE_Q: q [B,T,D,S,4]; Sq [B,T,D,4]; Dq strided [B,T,D]
  const void* q;
  const void* Sq;
  const void* Dq;
  int64_t d_sb, d_st, d_sd;
  // both
  const void* Bm;
  const void* Cm;
  const void* h0;
  void* y;
  void* h_last;
  // Optional fp32 state checkpoints [B, ceil(T/ckpt_every), D, S, 4]: the state
  // at the last step of every chunk of ckpt_every steps (for the backward).
  float* h_ckpt;
  int64_t ckpt_every;
  int64_t batch, T, Dm, S;
  float eps;
  // Chunked walk (MODE_DL inference, ssm_chunk.hpp): the T axis in n_chunks
  // chunks of chunk_len steps (the last may be shorter), one row of blocks per
  // (chunk, batch); chunk c > 0 starts from the state at the end of chunk c-1,
  // h_chunk[b, c-1] (fp32 [B, n_chunks - 1, D, S, 4]). n_chunks 1 (chunk_len
  // 0 or T) is the whole walk from h0.
  int64_t chunk_len = 0;
  int64_t n_chunks = 1;
  const float* h_chunk = nullptr;
};

template <typename T, int MODE, int KPL>
struct Step;

template <typename T, int KPL>
struct Step<T, MODE_DL, KPL> {
  Raw<T, 1> delta, s;
  Raw<T, 4 * KPL> B, C;
};

template <typename T, int KPL>
struct Step<T, MODE_Q, KPL> {
  Raw<T, 4 * KPL> q, B, C;
  Raw<T, 4> S;
  Raw<T, 1> D;
};

// Sum `acc` over the G lanes of a group (G a power of two, groups aligned in
// the wave). Returns, in v[0..NC), the components this lane ends up holding,
// and the index of the first of them in c0 (they are consecutive).
//   G == 1: all four, G == 2: two, G >= 4: one (component 2*(lane&1) + ((lane>>1)&1)),
// valid in the group's first four lanes (for G <= 16 in every lane).
template <int G>
__device__ inline int group_reduce(const quat& acc, int lane, float (&v)[4], int& c0) {
  if constexpr (G == 1) {
    v[0] = acc.w; v[1] = acc.x; v[2] = acc.y; v[3] = acc.z;
    c0 = 0;
    return 4;
  } else {
    const bool odd = lane & 1;
    // Stage 1 (lane ^ 1): even lanes keep components (0,1), odd lanes keep
    // (2,3); each adds the partner's copy of the pair it keeps.
    const float s0 = odd ? acc.w : acc.y;
    const float s1 = odd ? acc.x : acc.z;
    float k0 = odd ? acc.y : acc.w;
    float k1 = odd ? acc.z : acc.x;
    k0 += lane_xor1(s0);
    k1 += lane_xor1(s1);
    if constexpr (G == 2) {
      v[0] = k0; v[1] = k1;
      c0 = odd ? 2 : 0;
      return 2;
    } else {
      // Stage 2 (lane ^ 2): lanes with bit 1 clear keep the first of the pair.
      const bool hi = lane & 2;
      const float snd = hi ? k0 : k1;
      float kk = hi ? k1 : k0;
      kk += lane_xor2(snd);
      // Lanes holding the same component are 4 apart from here on.
      if constexpr (G == 8) kk += __shfl_xor(kk, 4);
      if constexpr (G >= 16) {
        kk += row_rot4(kk);
        kk += row_rot8(kk);
      }
      // Across rows the total lands in the group's first row, which holds the
      // writer lanes (j < 4).
      if constexpr (G >= 32) kk = sum_row_pair_to_even(kk);
      if constexpr (G == 64) kk = sum_halves_to_low(kk);
      v[0] = kk;
      c0 = (odd ? 2 : 0) + (hi ? 1 : 0);
      return 1;
    }
  }
}

__device__ inline float softplus_f(float x) {
  // torch.nn.functional.softplus with beta = 1, threshold = 20.
  return x > 20.f ? x : log1pf(expf(x));
}

// Per-(d,k) constants of the Cayley closed form for Lambda = (a, v):
// a = -softplus(alpha), v = tanh(imag), n2 = |Lambda|^2 / 4.
struct LamConst {
  float a, n2, v0, v1, v2;
};

__device__ inline LamConst lam_const(const float* lam_alpha, const float* lam_imag, int64_t dk) {
  LamConst c;
  c.a = -softplus_f(lam_alpha[dk]);
  c.v0 = tanhf(lam_imag[dk * 3 + 0]);
  c.v1 = tanhf(lam_imag[dk * 3 + 1]);
  c.v2 = tanhf(lam_imag[dk * 3 + 2]);
  c.n2 = 0.25f * (c.a * c.a + c.v0 * c.v0 + c.v1 * c.v1 + c.v2 * c.v2);
  return c;
}

// q = Cayley(dl * Lambda) = ((1 - dl^2 n2) / N, dl v / N), N = max(1 - dl a + dl^2 n2, eps).
// The forward kernel and the backward's recompute share this code, so both
// produce the same q.
// c receives dl / max(N, eps), the factor on v: q = q.w + c v.
__device__ inline quat cayley_step_c(float dl, float dl2, const LamConst& L, float eps, float& c) {
  float N = fmaf(dl2, L.n2, fmaf(-dl, L.a, 1.f));
  N = fmaxf(N, eps);
  const float r = __builtin_amdgcn_rcpf(N);
  c = dl * r;
  return quat{fmaf(-dl2, L.n2, 1.f) * r, c * L.v0, c * L.v1, c * L.v2};
}

__device__ inline quat cayley_step(float dl, float dl2, const LamConst& L, float eps) {
  float c;
  return cayley_step_c(dl, dl2, L, eps, c);
}

// h_t = q (x) h_{t-1} + s * B
__device__ inline quat state_step(const quat& q, const quat& h, float sv, const quat& Bk) {
  quat hn{sv * Bk.w, sv * Bk.x, sv * Bk.y, sv * Bk.z};
  qmul_acc(hn, q, h);
  return hn;
}

// FULL: S == KPL * G, so every lane of a group owns real states.
// SYNC: 0 = waves run freely; 1 = block barrier after every step; 2 = after
// every PF steps.
template <typename T, int MODE, int KPL, int G, int PF, int NT, bool FULL, int SYNC>
__global__ __launch_bounds__(NT) void ssm_scan_kernel(SsmArgs a) {
  static_assert((G & (G - 1)) == 0 && G <= 64 && NT % 64 == 0 && NT % G == 0,
                "G must be a power of two <= 64 dividing the block");
  constexpr int GPB = NT / G;  // groups (d's) per block
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int j = tid & (G - 1);
  int64_t bx, by;
  xcd_block(bx, by);
  // Block row by = chunk * batch + b (one chunk, the whole walk, unless chunked).
  const int chunk = a.n_chunks > 1 ? (int)(by / a.batch) : 0;
  const int64_t b = a.n_chunks > 1 ? by - (int64_t)chunk * a.batch : by;
  const int64_t d_raw = bx * GPB + tid / G;
  const bool gvalid = d_raw < a.Dm;
  const int64_t d = gvalid ? d_raw : a.Dm - 1;
  // Lane j owns KPL states. Where they take 32 bytes of B and of C per step
  // (four 16-bit or two fp32 states), or are two 16-bit states, and S == KPL * G,
  // they come as two pieces of KPL / 2 consecutive states half a (b, d) row
  // apart, k0 + [0, KPL / 2) and k0 + S / 2 + [0, KPL / 2) with k0 = j * KPL / 2
  // (SPLIT): each load instruction of a wave then reads whole 128-byte lines,
  // which lets the loads of B and C stream with the NT cache policy. (With one
  // contiguous 32-byte run per lane, each instruction reads half of every line
  // it touches, and NT loads measured 11 % slower at config 3.) For two 16-bit
  // states the pieces are 8 bytes of B and C, and one state (16 bytes of fp32)
  // of the training walk's checkpoints, so each checkpoint store instruction
  // writes whole lines too: training walk at config 4 2.70-2.75 -> 2.58-2.63 ms
  // (fp16), 2.78-2.79 -> 2.63-2.64 ms (bf16), same buffers, against contiguous
  // two-state lanes with NT loads. Otherwise the KPL states are consecutive
  // from k0 = j * KPL.
  constexpr bool SPLIT =
      FULL && (KPL * 4 * (int)sizeof(T) == 32 || (KPL == 2 && sizeof(T) == 2));
  constexpr int PIECE = SPLIT ? KPL / 2 : KPL;  // consecutive states per piece
  int k0 = j * PIECE;
  const bool kvalid = FULL || k0 < a.S;
  if (!kvalid) k0 = (int)a.S - KPL;
  // k of the lane's state kk.
  const int half_s = (int)a.S / 2;
  auto kof = [&](int kk) -> int {
    if constexpr (SPLIT) return kk >= PIECE ? k0 + half_s + (kk - PIECE) : k0 + kk;
    return k0 + kk;
  };
  // Loads of B, C (and q): whole lines per instruction (8- or 16-byte lanes, or
  // split 32-byte lanes) stream with the NT policy. Measured against the
  // previous kernel (contiguous lanes, cached loads) on the same buffers (bf16
  // unless noted): config-3 inference walk 2.09-2.17 -> 1.97-2.11 ms over three
  // allocations; training walk at config 4 2.87-2.90 -> 2.73-2.76 ms (fp16) and
  // 2.76 -> 2.69 ms; q form B4 T1024 1.63 -> 1.56 ms; B2 S128 2.16 -> 2.10 ms;
  // one-state lanes B2 T2048 d1536 S64 1.21 -> 1.16 ms, B4 S16 0.849 -> 0.841,
  // B1 unchanged (0.90 ms).
  constexpr int kPieceBytes = PIECE * 4 * (int)sizeof(T);
  constexpr int LOAD_AUX = (kPieceBytes == 8 || kPieceBytes == 16) ? 2 : 0;
  // Bytes from piece to piece: S / 2 states.
  constexpr int LOAD_STRIDE = SPLIT ? (KPL / 2) * 4 * (int)sizeof(T) * G : 16;

  // Step counters are 32-bit (the host checks T): gfx9's scalar unit has no
  // 64-bit compares, and 64-bit ones would run on the VALU every step.
  const int Tn = (int)a.T;
  // This block's steps: [tb, tb + Tw).
  const int Lc = a.n_chunks > 1 ? (int)a.chunk_len : Tn;
  const int tb = chunk * Lc;
  const int Tw = Tn - tb < Lc ? Tn - tb : Lc;
  const int64_t rowBC = a.Dm * a.S * 4;  // elements per (b, t) slice of B, C, q
  const int64_t rowTok = a.Dm;           // elements per (b, t) slice of delta, s
  // Byte offsets of this lane inside one (b, t) slice (the host checks that a
  // slice, and the strided D vector, stay below 2 GiB).
  const uint32_t offBC = (uint32_t)((d * a.S + k0) * 4 * (int64_t)sizeof(T));
  const uint32_t offTok = (uint32_t)(d * (int64_t)sizeof(T));
  const uint32_t offQ4 = (uint32_t)(d * 4 * (int64_t)sizeof(T));
  const uint32_t offD = (uint32_t)(d * a.d_sd * (int64_t)sizeof(T));

  // Per-(d,k) constants of the Cayley closed form (MODE_DL).
  LamConst lam[KPL];
  float dskip = 0.f;
  if constexpr (MODE == MODE_DL) {
#pragma unroll
    for (int kk = 0; kk < KPL; ++kk) lam[kk] = lam_const(a.lam_alpha, a.lam_imag, d * a.S + kof(kk));
    dskip = a.dvec[d];
  }

  // States. The block's form (MODE_DL) takes and returns the state in fp32,
  // the precision it is carried in here, so a walk split into pieces (the
  // recurrent decode) equals the whole walk; the q form keeps the reference's
  // convention of a state in the operands' dtype (ssm_fused.py:297-298).
  using HT = typename std::conditional<MODE == MODE_DL, float, T>::type;
  quat h[KPL];
#pragma unroll
  for (int kk = 0; kk < KPL; ++kk) h[kk] = quat{0.f, 0.f, 0.f, 0.f};
  // The lane's states in a [.., S, 4] state tensor, (b, d) row `r` (in units of
  // S states): one run of KPL states, or the two pieces of a SPLIT lane. (The
  // unsplit loads are written out at their two call sites: through this lambda
  // the 1024-thread one-lane-per-(b, d) kernel needed one VGPR more than its
  // 128 and spilled.)
  auto load_split_states = [&](const auto* p, int64_t r) {
    using ST = typename std::remove_cv<typename std::remove_pointer<decltype(p)>::type>::type;
#pragma unroll
    for (int pc = 0; pc < 2; ++pc) {
      float e[4 * PIECE];
      load_vec<ST, 4 * PIECE>(p + (r * a.S + kof(pc * PIECE)) * 4, e);
#pragma unroll
      for (int kk = 0; kk < PIECE; ++kk) h[pc * PIECE + kk] = quat_from(&e[4 * kk]);
    }
  };
  auto store_states = [&](auto* p, int64_t r, auto stream) {
    using ST = typename std::remove_pointer<decltype(p)>::type;
    constexpr bool NTS = decltype(stream)::value;
    float e[4 * KPL];
#pragma unroll
    for (int kk = 0; kk < KPL; ++kk) {
      e[4 * kk + 0] = h[kk].w; e[4 * kk + 1] = h[kk].x;
      e[4 * kk + 2] = h[kk].y; e[4 * kk + 3] = h[kk].z;
    }
    if constexpr (SPLIT) {
#pragma unroll
      for (int pc = 0; pc < 2; ++pc) {
        float f[4 * PIECE];
#pragma unroll
        for (int i = 0; i < 4 * PIECE; ++i) f[i] = e[4 * PIECE * pc + i];
        store_vec<ST, 4 * PIECE, NTS>(p + (r * a.S + kof(pc * PIECE)) * 4, f);
      }
    } else {
      store_vec<ST, 4 * KPL, NTS>(p + (r * a.S + k0) * 4, e);
    }
  };
  if (chunk > 0) {
    // The state at the end of the previous chunk (fp32, from the carry prefix).
    if constexpr (SPLIT) {
      load_split_states(a.h_chunk, (b * (a.n_chunks - 1) + chunk - 1) * a.Dm + d);
    } else {
      float e[4 * KPL];
      load_vec<float, 4 * KPL>(
          a.h_chunk + (((b * (a.n_chunks - 1) + chunk - 1) * a.Dm + d) * a.S + k0) * 4, e);
#pragma unroll
      for (int kk = 0; kk < KPL; ++kk) h[kk] = quat_from(&e[4 * kk]);
    }
  } else if (a.h0) {
    if constexpr (SPLIT) {
      load_split_states((const HT*)a.h0, b * a.Dm + d);
    } else {
      float e[4 * KPL];
      load_vec<HT, 4 * KPL>((const HT*)a.h0 + ((b * a.Dm + d) * a.S + k0) * 4, e);
#pragma unroll
      for (int kk = 0; kk < KPL; ++kk) h[kk] = quat_from(&e[4 * kk]);
    }
  }

  // Loads of step t into a ring slot. t is wave-uniform: each tensor's slice
  // base goes into a buffer descriptor (SGPRs) and the lane supplies only its
  // 32-bit byte offset inside the slice.
  auto load_step = [&](Step<T, MODE, KPL>& st, int t) {
    const int64_t rt = b * Tn + t;
    if constexpr (MODE == MODE_DL) {
      raw_load_buf<T, 1>(buf_rsrc((const T*)a.delta + rt * rowTok), offTok, st.delta);
      raw_load_buf<T, 1>(buf_rsrc((const T*)a.s + rt * rowTok), offTok, st.s);
    } else {
      raw_load_buf<T, 4>(buf_rsrc((const T*)a.Sq + rt * rowTok * 4), offQ4, st.S);
      raw_load_buf<T, 1>(buf_rsrc((const T*)a.Dq + b * a.d_sb + (int64_t)t * a.d_st), offD, st.D);
      raw_load_buf<T, 4 * KPL, LOAD_AUX, LOAD_STRIDE>(buf_rsrc((const T*)a.q + rt * rowBC), offBC,
                                                      st.q);
    }
    raw_load_buf<T, 4 * KPL, LOAD_AUX, LOAD_STRIDE>(buf_rsrc((const T*)a.Bm + rt * rowBC), offBC,
                                                    st.B);
    raw_load_buf<T, 4 * KPL, LOAD_AUX, LOAD_STRIDE>(buf_rsrc((const T*)a.Cm + rt * rowBC), offBC,
                                                    st.C);
  };

  Step<T, MODE, KPL> ring[PF];
  const int t_last = tb + Tw - 1;

  const bool writer = gvalid && (G < 4 || j < 4);
  const int64_t rowY = a.Dm * 4;
  const uint32_t offY = (uint32_t)(d * 4 * (int64_t)sizeof(T));
  // Checkpoint schedule (scalar): the next step whose state is saved. A chunk
  // of the time-chunked walk starts on a checkpoint boundary (the host keeps
  // chunk_len a multiple of ckpt_every), so its first checkpoint is the one
  // that ends tb + ckpt_every - 1.
  const int ckpt_every = (int)a.ckpt_every;
  const int64_t n_ckpt = a.h_ckpt ? (Tn + ckpt_every - 1) / ckpt_every : 0;
  int next_ckpt = a.h_ckpt ? (tb + ckpt_every - 1 < Tn ? tb + ckpt_every - 1 : Tn - 1) : -1;
  int64_t ckpt_idx = a.h_ckpt ? tb / ckpt_every : 0;

  // One step t from ring slot cur.
  auto walk_step = [&](auto refill, Step<T, MODE, KPL>& cur, int t) {
    constexpr bool REFILL = decltype(refill)::value;
    quat acc{0.f, 0.f, 0.f, 0.f};
    float sv = 0.f;
    float Sv[4] = {0.f, 0.f, 0.f, 0.f};
    float Dv = 0.f;
    if constexpr (MODE == MODE_DL) {
      const float dl = raw_get(cur.delta, 0);
      sv = raw_get(cur.s, 0);
      const float dl2 = dl * dl;
#pragma unroll
      for (int kk = 0; kk < KPL; ++kk) {
        const quat qd = cayley_step(dl, dl2, lam[kk], a.eps);
        h[kk] = state_step(qd, h[kk], sv, raw_quat(cur.B, kk));
        qmul_acc(acc, raw_quat(cur.C, kk), h[kk]);
      }
    } else {
      const quat Sq = raw_quat(cur.S, 0);
      Sv[0] = Sq.w; Sv[1] = Sq.x; Sv[2] = Sq.y; Sv[3] = Sq.z;
      Dv = raw_get(cur.D, 0);
#pragma unroll
      for (int kk = 0; kk < KPL; ++kk) {
        const quat qk = raw_quat(cur.q, kk);
        quat hn = qmul(raw_quat(cur.B, kk), Sq);
        qmul_acc(hn, qk, h[kk]);
        h[kk] = hn;
        qmul_acc(acc, raw_quat(cur.C, kk), hn);
      }
    }
    // Refill the consumed slot with step t + PF (clamped: the last group
    // re-reads the last step, which keeps the loads unconditional).
    if constexpr (REFILL) {
      const int tn = t + PF;
      load_step(cur, tn <= t_last ? tn : t_last);
    }
    if constexpr (!FULL) {
      if (!kvalid) acc = quat{0.f, 0.f, 0.f, 0.f};
    }

    float v[4];
    int c0;
    const int nc = group_reduce<G>(acc, lane, v, c0);
    if (writer) {
      const __amdgpu_buffer_rsrc_t ry = buf_rsrc((T*)a.y + (b * Tn + t) * rowY);
      if constexpr (MODE == MODE_DL) {
        if (c0 == 0) v[0] = fmaf(dskip, sv, v[0]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (e < nc) v[e] = fmaf(Dv, Sv[c0 + e], v[e]);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (e < nc) store_elem_buf<T>(ry, offY + (uint32_t)((c0 + e) * (int)sizeof(T)), v[e]);
    }
    if (a.h_ckpt && t == next_ckpt) {
      // Chunk t / ckpt_every ends here (or the sequence does).
      if (gvalid && kvalid) {
        // Nontemporal: the backward reads the checkpoints back after the rest of
        // the forward (the training forward measured 1-3 % faster at config 3).
        store_states(a.h_ckpt, (b * n_ckpt + ckpt_idx) * a.Dm + d, std::true_type{});
      }
      ++ckpt_idx;
      next_ckpt = next_ckpt + ckpt_every < Tn ? next_ckpt + ckpt_every : Tn - 1;
    }
    if constexpr (SYNC == 1) __syncthreads();
  };

  // Whole groups of PF steps run in a loop with no exit inside the group and
  // an unconditional prologue, so every path into the loop head has issued all
  // PF steps' loads in order: the wait for slot 0 leaves the later slots in
  // flight. (An exit inside the group, or prologue loads under conditions,
  // make the compiler assume at the loop head that slot 0 was loaded last,
  // and wait for every load in flight once per group.) The remaining steps,
  // and all of a walk shorter than PF, run in one guarded tail.
  //
  // Lanes that load 8 bytes of B and C per step (one 16-bit state) keep the
  // ring in flight across groups: measured at T 2048, D 1536, S 64 (bf16),
  // batch 1 1.00 -> 0.89 ms and batch 2 1.34 -> 1.25 ms. Lanes that load 16
  // bytes or more still wait for all their loads once per group, which
  // measured 0.5-1.5 % faster at the config-3 shape (B4 T2048 D1536 S64) than
  // keeping PF steps in flight, the same with 4 or 6 steps, and 0-2 % faster
  // for four states per lane (32 bytes) with 4 or 8 steps.
  constexpr bool DRAIN = KPL * 4 * sizeof(T) >= 16;
  // s_waitcnt vmcnt(0) with expcnt and lgkmcnt at their maxima (gfx9 fields:
  // vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[5:4] in bits [15:14]).
  constexpr int kWaitVm0 = 0x0F70;
  // Step counters below are relative to tb.
  int t0 = 0;
  if (Tw >= PF) {
    // The scheduling barriers keep the prologue's loads in slot order.
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      load_step(ring[i], tb + i);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (; t0 + PF <= Tw; t0 += PF) {
      if constexpr (DRAIN) __builtin_amdgcn_s_waitcnt(kWaitVm0);
#pragma unroll
      for (int i = 0; i < PF; ++i) walk_step(std::true_type{}, ring[i], tb + t0 + i);
      if constexpr (SYNC == 2) __syncthreads();
    }
  } else {
    // A walk shorter than PF (a decode step has T = 1) loads only its steps.
#pragma unroll
    for (int i = 0; i < PF; ++i)
      if (i < Tw) load_step(ring[i], tb + i);
  }
  if (t0 < Tw) {
#pragma unroll
    for (int i = 0; i < PF; ++i)
      if (t0 + i < Tw) walk_step(std::false_type{}, ring[i], tb + t0 + i);
    if constexpr (SYNC == 2) __syncthreads();
  }

  if (a.h_last && gvalid && kvalid && chunk == a.n_chunks - 1)
    store_states((HT*)a.h_last, b * a.Dm + d, std::false_type{});
}

// Steps of operands in flight per lane (six for four 16-bit states per lane:
// measured at config 3 against four and eight).
template <typename T, int KPL>
constexpr int ssm_prefetch() {
  return KPL * (int)sizeof(T) >= 8 ? (sizeof(T) == 2 && KPL == 4 ? 6 : 4) : 8;
}

template <typename T, int MODE, int KPL, int G, int PF = ssm_prefetch<T, KPL>(),
          int NT = kSsmThreads, int SYNC = 0>
int launch_ssm_g(const SsmArgs& a, hipStream_t s) {
  constexpr int GPB = NT / G;
  const int64_t gx = (a.Dm + GPB - 1) / GPB;
  const int64_t gy = a.batch * a.n_chunks;  // (chunk, batch) rows
  if (gx > 0x7fffffffLL || gy > 65535) return MQC_E_LIMIT;
  const dim3 grid((unsigned)gx, (unsigned)gy);
  if (a.S == (int64_t)KPL * G)
    ssm_scan_kernel<T, MODE, KPL, G, PF, NT, true, SYNC><<<grid, dim3(NT), 0, s>>>(a);
  else
    ssm_scan_kernel<T, MODE, KPL, G, PF, NT, false, SYNC><<<grid, dim3(NT), 0, s>>>(a);
  return launch_status();
}

// Block shape. The waves of a block run in lockstep (a barrier after every
// step), so at any moment a block reads one contiguous span of each (b, t)
// slice of B and C instead of scattered 1 KiB pieces at drifting t: DRAM row
// locality, measured on MI355X at 4.76 -> 5.44 TB/s for the config-3 shape.
// Every block walks all T steps, so the busiest CU sets the time: the shape is
// the one that minimises ceil(blocks / CUs) * waves per block, the waves of
// work that CU carries; ties go to 768, 1024, 512, 256 threads in that order
// (768 measured best where it fills the machine exactly). Measured at B4 T2048
// S64 (bf16): d_inner 1536: 768 threads 2.33 ms, 1024 2.55, 512 2.62;
// d_inner 2048: 768 threads (344 blocks, a second round for 88 CUs) 3.81 ms,
// 1024 (256 blocks) 3.04, 512 3.18; d_inner 1024 (one state per lane):
// 768 threads 2.53 ms, 1024 1.70.
constexpr int kCUs = 256;  // MI355X compute units

inline int64_t busiest_cu_waves(const SsmArgs& a, int G, int NT) {
  const int64_t gpb = NT / G;
  const int64_t blocks = a.batch * a.n_chunks * ((a.Dm + gpb - 1) / gpb);
  return (blocks + kCUs - 1) / kCUs * (NT / 64);
}

// The largest block whose lanes get the kernel's registers without spilling
// to scratch (NT threads leave 512 / (NT / 256) VGPRs per lane), from the
// register counts of the compiled kernels: the materialised-q form carries
// q, S and D in the ring besides B and C, and four states per lane carry twice
// the operands of two.
template <typename T, int MODE, int KPL>
constexpr int ssm_max_threads() {
  if constexpr (MODE == MODE_DL) return KPL <= 2 ? 1024 : 512;
  if constexpr (sizeof(T) == 2) return KPL == 1 ? 1024 : (KPL == 2 ? 768 : 512);
  return KPL <= 2 ? 768 : 256;
}

template <typename T, int MODE, int KPL, int G>
int launch_ssm_shape(const SsmArgs& a, hipStream_t s) {
  constexpr int PF = ssm_prefetch<T, KPL>();
  constexpr int kMaxNT = ssm_max_threads<T, MODE, KPL>();
  int best = 256;
  if constexpr (G <= 64) {
    // 384 threads (6 waves) only for lanes with 32 bytes of each operand per
    // step (four 16-bit or two fp32 states), where it puts one block on every
    // CU at config 3.
    const int order[5] = {768, 1024, 512, 384, 256};
    int64_t best_w = -1;
    for (int nt : order) {
      if (nt % G != 0 || nt > kMaxNT || (nt == 384 && KPL * sizeof(T) != 8)) continue;
      const int64_t w = busiest_cu_waves(a, G, nt);
      if (best_w < 0 || w < best_w) {
        best_w = w;
        best = nt;
      }
    }
  }
  switch (best) {
    case 768:
      if constexpr (kMaxNT >= 768) return launch_ssm_g<T, MODE, KPL, G, PF, 768, 1>(a, s);
      break;
    case 1024:
      if constexpr (kMaxNT >= 1024) return launch_ssm_g<T, MODE, KPL, G, PF, 1024, 1>(a, s);
      break;
    case 512:
      if constexpr (kMaxNT >= 512) return launch_ssm_g<T, MODE, KPL, G, PF, 512, 1>(a, s);
      break;
    case 384:
      if constexpr (KPL * sizeof(T) == 8 && kMaxNT >= 384) return launch_ssm_g<T, MODE, KPL, G, PF, 384, 1>(a, s);
      break;
    default:
      break;
  }
  return launch_ssm_g<T, MODE, KPL, G, PF, 256, 1>(a, s);
}

template <typename T, int MODE, int KPL>
int launch_ssm_kpl(const SsmArgs& a, hipStream_t s) {
  const int64_t per = (a.S + KPL - 1) / KPL;  // lanes needed per (b, d)
  if (per <= 1) return launch_ssm_shape<T, MODE, KPL, 1>(a, s);
  if (per <= 2) return launch_ssm_shape<T, MODE, KPL, 2>(a, s);
  if (per <= 4) return launch_ssm_shape<T, MODE, KPL, 4>(a, s);
  if (per <= 8) return launch_ssm_shape<T, MODE, KPL, 8>(a, s);
  if (per <= 16) return launch_ssm_shape<T, MODE, KPL, 16>(a, s);
  if (per <= 32) return launch_ssm_shape<T, MODE, KPL, 32>(a, s);
  if (per <= 64) return launch_ssm_shape<T, MODE, KPL, 64>(a, s);
  return MQC_E_LIMIT;
}

// Lane width: 16-byte loads of B and C where the layout allows (two states
// per lane for 16-bit storage, one for fp32), wider lanes for d_state > 64.
// KPL states per lane need d_state % KPL == 0 (lanes past the last k are
// clamped onto the last KPL states).
// What every launch of the walk needs of its arguments, checked on the host
// before any kernel runs (the chunked walk calls it before its carry launch).
template <typename T, int MODE>
int ssm_check(const SsmArgs& a) {
  // Per-(b, t) slices (and the strided D vector) are addressed with 32-bit lane
  // offsets; step counters are 32-bit.
  if (a.Dm * a.S * 4 * (int64_t)sizeof(T) >= ((int64_t)1 << 31)) return MQC_E_LIMIT;
  if (a.T >= ((int64_t)1 << 30) || (a.h_ckpt && (a.ckpt_every < 1 || a.ckpt_every >= (1 << 30))))
    return MQC_E_LIMIT;
  if (MODE == MODE_Q && (a.d_sd < 0 || (a.Dm - 1) * a.d_sd * (int64_t)sizeof(T) >= ((int64_t)1 << 31)))
    return MQC_E_LIMIT;
  const uintptr_t qa = 4 * sizeof(T);
  // The state (h0, h_last) is fp32 in MODE_DL, the operands' dtype in MODE_Q.
  const uintptr_t ha = MODE == MODE_DL ? 16 : qa;
  if (!aligned(a.Bm, qa) || !aligned(a.Cm, qa) || !aligned(a.y, sizeof(T)) ||
      (MODE == MODE_Q && (!aligned(a.q, qa) || !aligned(a.Sq, qa) || !aligned(a.Dq, sizeof(T)))) ||
      (a.h0 && !aligned(a.h0, ha)) || (a.h_last && !aligned(a.h_last, ha)))
    return MQC_E_ALIGN;
  return MQC_OK;
}

template <typename T, int MODE>
int launch_ssm(const SsmArgs& a, hipStream_t s) {
  // T == 0 with h_last still launches: the walk is empty and the kernel writes
  // h_last from h0 (or zeros).
  if (a.batch == 0 || a.Dm == 0 || (a.T == 0 && !a.h_last)) return MQC_OK;
  const int chk = ssm_check<T, MODE>(a);
  if (chk != MQC_OK) return chk;
  auto wide_ok = [&](int kpl) {
    const uintptr_t al = kpl * 4 * sizeof(T) >= 16 ? 16 : kpl * 4 * sizeof(T);
    const uintptr_t hal = MODE == MODE_DL ? 16 : al;
    return a.S % kpl == 0 && aligned(a.Bm, al) && aligned(a.Cm, al) &&
           (MODE == MODE_DL || aligned(a.q, al)) && (!a.h0 || aligned(a.h0, hal)) &&
           (!a.h_last || aligned(a.h_last, hal));
  };
  if constexpr (sizeof(T) == 2) {
    // Two states per lane fill the machine at config 3 (3072 waves, 12 per CU:
    // 2.34 ms against 2.74 with one state per lane). With fewer waves than that
    // (small batch x d_inner), one state per lane doubles the lanes: measured at
    // T 2048, D 1536, S 64: batch 1 1.063 -> 1.001 ms, batch 2 1.391 -> 1.340 ms.
    const int64_t waves_kpl2 = a.batch * a.n_chunks * a.Dm * ((a.S + 1) / 2) / 64;
    if (a.S <= 64 && waves_kpl2 < 12 * kCUs) return launch_ssm_kpl<T, MODE, 1>(a, s);
    // Four states per lane (32 bytes of B and C per lane and step, 384-thread
    // blocks, six steps in flight) for the inference walk: fewer k-sum and
    // per-step instructions per state and half the waves at each barrier.
    // Measured at T 2048, S 64 (bf16), same buffers, against two states per
    // lane: B4 d_inner 1536 2.288 -> 2.221 ms, B8 d1536 4.765 -> 4.724,
    // B4 d2048 3.126 -> 3.088, B4 d3072 4.381 -> 4.319, B16 d768 4.383 -> 4.334,
    // B2 d3072 2.299 -> 2.229; B6 d1536 4.074 -> 4.131. The training walk
    // (checkpoints) measured 36 % slower with four states and keeps two.
    if constexpr (MODE == MODE_DL) {
      if (a.S <= 64 && !a.h_ckpt && wide_ok(4)) return launch_ssm_kpl<T, MODE, 4>(a, s);
    }
    if (a.S <= 128 && wide_ok(2)) return launch_ssm_kpl<T, MODE, 2>(a, s);
    if (a.S <= 64) return launch_ssm_kpl<T, MODE, 1>(a, s);
    if (a.S <= 256 && wide_ok(4)) return launch_ssm_kpl<T, MODE, 4>(a, s);
    return MQC_E_LIMIT;
  } else {
    // fp32: two states per lane (32 bytes of each operand per lane and step)
    // once that still gives 6 waves per CU, except in the training walk.
    // Measured at S 64, same buffers, against one state per lane: delta-lambda
    // form B4 T2048 d1536 4.66 -> 4.45 ms, B8 T1024 d1536 4.75 -> 4.57,
    // B4 T1024 d3072 4.51 -> 4.37, B2 T2048 d1536 2.34 -> 2.33; q form
    // B4 T1024 d1536 3.38 -> 3.26, B8 T512 d1536 3.46 -> 3.31.
    if (a.S <= 64 && !a.h_ckpt && wide_ok(2) &&
        a.batch * a.n_chunks * a.Dm * (a.S / 2) / 64 >= 6 * kCUs)
      return launch_ssm_kpl<T, MODE, 2>(a, s);
    if (a.S <= 64) return launch_ssm_kpl<T, MODE, 1>(a, s);
    if (a.S <= 128 && wide_ok(2)) return launch_ssm_kpl<T, MODE, 2>(a, s);
    if (a.S <= 256 && wide_ok(4)) return launch_ssm_kpl<T, MODE, 4>(a, s);
    return MQC_E_LIMIT;
  }
}

// One translation unit per storage type instantiates these (ssm_scan_*.hip),
// so the three compile in parallel.
extern template int launch_ssm<float, MODE_DL>(const SsmArgs&, hipStream_t);
extern template int launch_ssm<float, MODE_Q>(const SsmArgs&, hipStream_t);
extern template int launch_ssm<bf16_t, MODE_DL>(const SsmArgs&, hipStream_t);
extern template int launch_ssm<bf16_t, MODE_Q>(const SsmArgs&, hipStream_t);
extern template int launch_ssm<f16_t, MODE_DL>(const SsmArgs&, hipStream_t);
extern template int launch_ssm<f16_t, MODE_Q>(const SsmArgs&, hipStream_t);

}  // namespace mqc
