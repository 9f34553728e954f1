#pragma once
// Time-chunked walk of the block's fused quaternion SSM (delta-lambda form).
//
// The whole walk (ssm_scan.hpp) gives every (b, d, k) lane one sequential
// pass over all T steps, so its parallelism is batch * d_inner * d_state
// states. Where that is too few to keep the CUs busy (batch 1, small
// d_state), the T axis is cut into n_chunks chunks of L steps and the chunks
// run side by side. The recurrence of one lane is an affine map per step,
//   h_t = q_t (x) h_{t-1} + s_t B_t  =  M_t(h_{t-1}),
// so chunk c as a whole is M_c(h) = P_c (x) h + H_c with P_c the product of
// its q's (later factors on the left) and H_c its end state from zero.
// Composing two chunks keeps the later one on the left:
//   (P2, H2) o (P1, H1) = (P2 (x) P1, P2 (x) H1 + H2).
// Three launches:
//   1. ssm_chunk_agg_kernel: every chunk but the last walks its L steps from
//      zero, reading delta, s and B, and stores (P_c, H_c).
//   2. ssm_carry_prefix_kernel: an inclusive scan over the chunks of each lane,
//      one wave segment per lane with the chunks on consecutive lanes, combined
//      by DPP row shifts and row broadcasts in the order above; h0 is folded
//      into the first chunk. Lane c leaves the state at the end of chunk c.
//   3. ssm_scan_kernel (ssm_scan.hpp) walks every chunk from that state and
//      writes y (and h_last from the last chunk).
// The chunked walk reads B twice for all chunks but the last (launches 1 and
// 3): 1.25-1.5x the whole walk's bytes for 2-4 chunks, bought back where the
// whole walk is latency-bound.
//
// In this form every q_t of a lane is q = qw + c v with the lane's fixed pure
// quaternion v = Lambda_vec (ssm_scan.hpp, cayley_step), so every product of
// them is P = Pa + Pb v (v (x) v = -|v|^2): two floats per lane, and
//   (Pa + Pb v)(Pa' + Pb' v) = (Pa Pa' - Pb Pb' |v|^2) + (Pa Pb' + Pb Pa') v.
#include "ssm_scan.hpp"

namespace mqc {

// Largest d_state of the chunked walk (one wave segment of lanes per (b, d)).
constexpr int kChunkMaxState = 64;

// P (x) h for P = pa + pb v (v pure, per lane).
__device__ inline quat vplane_mul(float pa, float pb, const LamConst& L, const quat& h) {
  const quat v{0.f, L.v0, L.v1, L.v2};
  const quat vh = qmul(v, h);
  return quat{fmaf(pa, h.w, pb * vh.w), fmaf(pa, h.x, pb * vh.x), fmaf(pa, h.y, pb * vh.y),
              fmaf(pa, h.z, pb * vh.z)};
}

template <typename T, int KPL>
struct AggStep {
  Raw<T, 1> delta, s;
  Raw<T, 4 * KPL> B;
};

// Launch 1. Grid (d-blocks, batch * (n_chunks - 1)); block row by = chunk *
// batch + b. Every chunk here is full (L steps): only the last chunk may be
// shorter, and it has no carry. Lockstep blocks (a barrier per step), as the
// whole walk, keep each block's reads of a (b, t) slice together.
// Hc: fp32 [B, n_chunks - 1, D, S, 4]; Pc: fp32 [B, n_chunks - 1, D, S, 2].
template <typename T, int KPL, int G, int PF, int NT, bool FULL>
__global__ __launch_bounds__(NT) void ssm_chunk_agg_kernel(SsmArgs a, float* Hc, float* Pc) {
  static_assert((G & (G - 1)) == 0 && G <= 64 && NT % 64 == 0 && NT % G == 0, "bad group");
  constexpr int GPB = NT / G;
  const int tid = threadIdx.x;
  const int j = tid & (G - 1);
  int64_t bx, by;
  xcd_block(bx, by);
  const int chunk = (int)(by / a.batch);
  const int64_t b = by - (int64_t)chunk * a.batch;
  const int64_t d_raw = bx * GPB + tid / G;
  const bool gvalid = d_raw < a.Dm;
  const int64_t d = gvalid ? d_raw : a.Dm - 1;
  int k0 = j * KPL;
  const bool kvalid = FULL || k0 < a.S;
  if (!kvalid) k0 = (int)a.S - KPL;

  const int Tn = (int)a.T;
  const int Lc = (int)a.chunk_len;
  const int tb = chunk * Lc;
  const int64_t rowBC = a.Dm * a.S * 4;
  const int64_t rowTok = a.Dm;
  const uint32_t offBC = (uint32_t)((d * a.S + k0) * 4 * (int64_t)sizeof(T));
  const uint32_t offTok = (uint32_t)(d * (int64_t)sizeof(T));

  LamConst lam[KPL];
  float vv[KPL];
  quat h[KPL];
  float pa[KPL], pb[KPL];
#pragma unroll
  for (int kk = 0; kk < KPL; ++kk) {
    lam[kk] = lam_const(a.lam_alpha, a.lam_imag, d * a.S + k0 + kk);
    vv[kk] = lam[kk].v0 * lam[kk].v0 + lam[kk].v1 * lam[kk].v1 + lam[kk].v2 * lam[kk].v2;
    h[kk] = quat{0.f, 0.f, 0.f, 0.f};
    pa[kk] = 1.f;
    pb[kk] = 0.f;
  }

  auto load_step = [&](AggStep<T, KPL>& st, int t) {
    const int64_t rt = b * Tn + t;
    raw_load_buf<T, 1>(buf_rsrc((const T*)a.delta + rt * rowTok), offTok, st.delta);
    raw_load_buf<T, 1>(buf_rsrc((const T*)a.s + rt * rowTok), offTok, st.s);
    // B with the NT cache policy where each instruction reads whole lines (8 or
    // 16 bytes per lane): B1 T2048 d1536 S64 chunked walk 0.770 -> 0.752 ms.
    raw_load_buf<T, 4 * KPL, (KPL * 4 * sizeof(T) <= 16 ? 2 : 0)>(
        buf_rsrc((const T*)a.Bm + rt * rowBC), offBC, st.B);
  };
  const int t_last = tb + Lc - 1;
  auto step = [&](auto refill, AggStep<T, KPL>& cur, int t) {
    constexpr bool REFILL = decltype(refill)::value;
    const float dl = raw_get(cur.delta, 0);
    const float sv = raw_get(cur.s, 0);
    const float dl2 = dl * dl;
#pragma unroll
    for (int kk = 0; kk < KPL; ++kk) {
      float c;  // q = q.w + c v
      const quat q = cayley_step_c(dl, dl2, lam[kk], a.eps, c);
      h[kk] = state_step(q, h[kk], sv, raw_quat(cur.B, kk));
      const float na = fmaf(q.w, pa[kk], -c * pb[kk] * vv[kk]);
      pb[kk] = fmaf(q.w, pb[kk], c * pa[kk]);
      pa[kk] = na;
    }
    if constexpr (REFILL) {
      const int tn = t + PF;
      load_step(cur, tn <= t_last ? tn : t_last);
    }
    __syncthreads();
  };

  AggStep<T, KPL> ring[PF];
  int t0 = 0;
  if (Lc >= PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      load_step(ring[i], tb + i);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (; t0 + PF <= Lc; t0 += PF) {
#pragma unroll
      for (int i = 0; i < PF; ++i) step(std::true_type{}, ring[i], tb + t0 + i);
    }
  } else {
#pragma unroll
    for (int i = 0; i < PF; ++i)
      if (i < Lc) load_step(ring[i], tb + i);
  }
  if (t0 < Lc) {
#pragma unroll
    for (int i = 0; i < PF; ++i)
      if (t0 + i < Lc) step(std::false_type{}, ring[i], tb + t0 + i);
  }

  if (gvalid && kvalid) {
    const int64_t base = ((b * (a.n_chunks - 1) + chunk) * a.Dm + d) * a.S + k0;
    float e[4 * KPL];
#pragma unroll
    for (int kk = 0; kk < KPL; ++kk) {
      e[4 * kk + 0] = h[kk].w; e[4 * kk + 1] = h[kk].x;
      e[4 * kk + 2] = h[kk].y; e[4 * kk + 3] = h[kk].z;
    }
    store_vec<float, 4 * KPL>(Hc + base * 4, e);
#pragma unroll
    for (int kk = 0; kk < KPL; ++kk) {
      Pc[(base + kk) * 2 + 0] = pa[kk];
      Pc[(base + kk) * 2 + 1] = pb[kk];
    }
  }
}

// One element of the carry scan: the map h -> P (x) h + H, P = pa + pb v.
struct ChunkMap {
  float pa, pb;
  quat H;
};

// later o earlier (the later map on the left).
__device__ inline ChunkMap compose(const ChunkMap& later, const ChunkMap& earlier, float vv,
                                   const LamConst& L) {
  ChunkMap r;
  r.pa = fmaf(later.pa, earlier.pa, -later.pb * earlier.pb * vv);
  r.pb = fmaf(later.pa, earlier.pb, later.pb * earlier.pa);
  const quat ph = vplane_mul(later.pa, later.pb, L, earlier.H);
  r.H = quat{ph.w + later.H.w, ph.x + later.H.x, ph.y + later.H.y, ph.z + later.H.z};
  return r;
}

// DPP move with an explicit fallback: lanes whose source is outside the
// pattern, or whose row is masked off, keep `old`.
template <int CTRL, int ROW_MASK>
__device__ inline float dpp_or(float old, float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, v), CTRL,
                                                               ROW_MASK, 0xF, false));
}

template <int CTRL, int ROW_MASK>
__device__ inline ChunkMap dpp_map(const ChunkMap& m) {
  ChunkMap r;
  r.pa = dpp_or<CTRL, ROW_MASK>(1.f, m.pa);
  r.pb = dpp_or<CTRL, ROW_MASK>(0.f, m.pb);
  r.H.w = dpp_or<CTRL, ROW_MASK>(0.f, m.H.w);
  r.H.x = dpp_or<CTRL, ROW_MASK>(0.f, m.H.x);
  r.H.y = dpp_or<CTRL, ROW_MASK>(0.f, m.H.y);
  r.H.z = dpp_or<CTRL, ROW_MASK>(0.f, m.H.z);
  return r;
}

// Launch 2. SEG consecutive lanes (a power of two <= 64, at least the number
// of carries when that is <= 64) own one (b, d, k); lane i of a segment holds
// chunk base + i. Inclusive scan within each 16-lane row by row shifts of 1,
// 2, 4, 8, then across rows by row_bcast:15 (rows 1 and 3 take lane 15 of the
// row before) and row_bcast:31 (rows 2 and 3 take lane 31), each composing the
// earlier prefix on the right. More than 64 carries take rounds of 64, the
// running state folded into the next round's first chunk. Every wave of the
// launch runs the same rounds (the count is uniform), so the cross-lane moves
// see the whole wave. Afterwards Hc[b, c] holds the state at the end of chunk
// c: the start of chunk c + 1.
template <int SEG>
__global__ __launch_bounds__(256) void ssm_carry_prefix_kernel(SsmArgs a, float* Hc, const float* Pc) {
  static_assert((SEG & (SEG - 1)) == 0 && SEG <= 64, "segment");
  constexpr int ROWSEG = SEG < 16 ? SEG : 16;
  const int lane = threadIdx.x & 63;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nstate = a.batch * a.Dm * a.S;
  const int64_t state_raw = gid / SEG;
  const bool valid = state_raw < nstate;
  const int64_t st = valid ? state_raw : nstate - 1;
  const int sl = (int)(gid & (SEG - 1));
  const int64_t b = st / (a.Dm * a.S);
  const int64_t dk = st - b * a.Dm * a.S;
  const int64_t d = dk / a.S;
  const LamConst L = lam_const(a.lam_alpha, a.lam_imag, dk);
  const float vv = L.v0 * L.v0 + L.v1 * L.v1 + L.v2 * L.v2;
  const int nc = (int)(a.n_chunks - 1);

  quat carry{0.f, 0.f, 0.f, 0.f};
  if (a.h0) {
    float e[4];
    load_vec<float, 4>((const float*)a.h0 + st * 4, e);
    carry = quat_from(e);
  }
  for (int base = 0; base < nc; base += SEG) {
    const int c = base + sl;
    const bool live = c < nc;
    const int64_t idx = ((b * nc + (live ? c : nc - 1)) * a.Dm + d) * a.S + (dk - d * a.S);
    ChunkMap m;
    if (live) {
      float e[4];
      load_vec<float, 4>(Hc + idx * 4, e);
      m.H = quat_from(e);
      m.pa = Pc[idx * 2 + 0];
      m.pb = Pc[idx * 2 + 1];
    } else {
      m.H = quat{0.f, 0.f, 0.f, 0.f};
      m.pa = 1.f;
      m.pb = 0.f;
    }
    if (sl == 0) {
      // The running state enters the segment's first chunk.
      const quat ph = vplane_mul(m.pa, m.pb, L, carry);
      m.H = quat{ph.w + m.H.w, ph.x + m.H.x, ph.y + m.H.y, ph.z + m.H.z};
    }
    // Within rows (and within segments shorter than a row).
    if constexpr (SEG > 1) {
      const ChunkMap e1 = dpp_map<0x111, 0xF>(m);  // row_shr:1
      if ((lane & (ROWSEG - 1)) >= 1) m = compose(m, e1, vv, L);
    }
    if constexpr (SEG > 2) {
      const ChunkMap e2 = dpp_map<0x112, 0xF>(m);  // row_shr:2
      if ((lane & (ROWSEG - 1)) >= 2) m = compose(m, e2, vv, L);
    }
    if constexpr (SEG > 4) {
      const ChunkMap e4 = dpp_map<0x114, 0xF>(m);  // row_shr:4
      if ((lane & (ROWSEG - 1)) >= 4) m = compose(m, e4, vv, L);
    }
    if constexpr (SEG > 8) {
      const ChunkMap e8 = dpp_map<0x118, 0xF>(m);  // row_shr:8
      if ((lane & (ROWSEG - 1)) >= 8) m = compose(m, e8, vv, L);
    }
    // Across rows.
    if constexpr (SEG > 16) {
      const ChunkMap r15 = dpp_map<0x142, 0xA>(m);  // row_bcast:15 into rows 1, 3
      if ((lane >> 4) & 1) m = compose(m, r15, vv, L);
    }
    if constexpr (SEG > 32) {
      const ChunkMap r31 = dpp_map<0x143, 0xC>(m);  // row_bcast:31 into rows 2, 3
      if (lane >= 32) m = compose(m, r31, vv, L);
    }
    if (valid && live) {
      const float e[4] = {m.H.w, m.H.x, m.H.y, m.H.z};
      store_vec<float, 4>(Hc + idx * 4, e);
    }
    if (base + SEG < nc) {
      // Only SEG == 64 takes more than one round: lane 63 ends the segment.
      auto last = [](float v) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
      };
      carry = quat{last(m.H.w), last(m.H.x), last(m.H.y), last(m.H.z)};
    }
  }
}

// Bytes of workspace the chunked walk needs: (P, H) of every chunk but the last.
inline int64_t ssm_chunk_workspace_bytes(int64_t batch, int64_t T, int64_t Dm, int64_t S,
                                         int64_t L) {
  if (L < 1 || T <= L) return 0;
  const int64_t nc = (T + L - 1) / L;
  return batch * (nc - 1) * Dm * S * (4 + 2) * (int64_t)sizeof(float);
}

template <typename T, int KPL, int G>
int launch_chunk_agg_g(const SsmArgs& a, float* Hc, float* Pc, hipStream_t s) {
  constexpr int NT = 256;
  constexpr int PF = ssm_prefetch<T, KPL>();
  constexpr int GPB = NT / G;
  const int64_t gx = (a.Dm + GPB - 1) / GPB;
  const int64_t gy = a.batch * (a.n_chunks - 1);
  if (gx > 0x7fffffffLL || gy > 65535) return MQC_E_LIMIT;
  const dim3 grid((unsigned)gx, (unsigned)gy);
  if (a.S == (int64_t)KPL * G)
    ssm_chunk_agg_kernel<T, KPL, G, PF, NT, true><<<grid, dim3(NT), 0, s>>>(a, Hc, Pc);
  else
    ssm_chunk_agg_kernel<T, KPL, G, PF, NT, false><<<grid, dim3(NT), 0, s>>>(a, Hc, Pc);
  return launch_status();
}

template <typename T, int KPL>
int launch_chunk_agg_kpl(const SsmArgs& a, float* Hc, float* Pc, hipStream_t s) {
  const int64_t per = (a.S + KPL - 1) / KPL;
  if (per <= 1) return launch_chunk_agg_g<T, KPL, 1>(a, Hc, Pc, s);
  if (per <= 2) return launch_chunk_agg_g<T, KPL, 2>(a, Hc, Pc, s);
  if (per <= 4) return launch_chunk_agg_g<T, KPL, 4>(a, Hc, Pc, s);
  if (per <= 8) return launch_chunk_agg_g<T, KPL, 8>(a, Hc, Pc, s);
  if (per <= 16) return launch_chunk_agg_g<T, KPL, 16>(a, Hc, Pc, s);
  if (per <= 32) return launch_chunk_agg_g<T, KPL, 32>(a, Hc, Pc, s);
  if (per <= 64) return launch_chunk_agg_g<T, KPL, 64>(a, Hc, Pc, s);
  return MQC_E_LIMIT;
}

template <int SEG>
int launch_carry_prefix(const SsmArgs& a, float* Hc, const float* Pc, hipStream_t s) {
  const int64_t threads = a.batch * a.Dm * a.S * SEG;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffffLL) return MQC_E_LIMIT;
  ssm_carry_prefix_kernel<SEG><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(a, Hc, Pc);
  return launch_status();
}

// The three launches of the chunked walk. a.chunk_len and a.n_chunks are set
// (n_chunks > 1); ws holds ssm_chunk_workspace_bytes; the caller has checked
// the arguments as for the whole walk, d_state <= kChunkMaxState and the
// launch limits below.
template <typename T>
int ssm_chunk_launch(const SsmArgs& a0, float* ws, hipStream_t s) {
  SsmArgs a = a0;
  // The walk's own argument checks, before the carry launch reads anything.
  const int chk = ssm_check<T, MODE_DL>(a);
  if (chk != MQC_OK) return chk;
  const int64_t nc = a.n_chunks - 1;
  float* Hc = ws;
  float* Pc = ws + a.batch * nc * a.Dm * a.S * 4;
  // States per lane of the carry walk: as many as still give 6 waves per CU.
  const int64_t rows = a.batch * nc;
  auto waves = [&](int kpl) { return rows * a.Dm * ((a.S + kpl - 1) / kpl) / 64; };
  auto fits = [&](int kpl) {
    const uintptr_t al = kpl * 4 * sizeof(T) >= 16 ? 16 : kpl * 4 * sizeof(T);
    return a.S % kpl == 0 && aligned(a.Bm, al) && waves(kpl) >= 6 * kCUs;
  };
  int st;
  if (sizeof(T) == 2 && fits(4))
    st = launch_chunk_agg_kpl<T, 4>(a, Hc, Pc, s);
  else if (fits(2))
    st = launch_chunk_agg_kpl<T, 2>(a, Hc, Pc, s);
  else
    st = launch_chunk_agg_kpl<T, 1>(a, Hc, Pc, s);
  if (st != MQC_OK) return st;
  if (nc <= 1) st = launch_carry_prefix<1>(a, Hc, Pc, s);
  else if (nc <= 2) st = launch_carry_prefix<2>(a, Hc, Pc, s);
  else if (nc <= 4) st = launch_carry_prefix<4>(a, Hc, Pc, s);
  else if (nc <= 8) st = launch_carry_prefix<8>(a, Hc, Pc, s);
  else if (nc <= 16) st = launch_carry_prefix<16>(a, Hc, Pc, s);
  else if (nc <= 32) st = launch_carry_prefix<32>(a, Hc, Pc, s);
  else st = launch_carry_prefix<64>(a, Hc, Pc, s);
  if (st != MQC_OK) return st;
  a.h_chunk = Hc;
  return launch_ssm<T, MODE_DL>(a, s);
}

extern template int ssm_chunk_launch<float>(const SsmArgs&, float*, hipStream_t);
extern template int ssm_chunk_launch<bf16_t>(const SsmArgs&, float*, hipStream_t);
extern template int ssm_chunk_launch<f16_t>(const SsmArgs&, float*, hipStream_t);

}  // namespace mqc
