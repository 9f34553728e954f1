// Backward of the block's fused quaternion SSM (delta-lambda form).
//
// Forward (ssm_scan.hpp), per lane (b, d, k):
//   q_t = Cayley(delta_t * Lambda)          Lambda = (-softplus(alpha), tanh(imag))
//   h_t = q_t (x) h_{t-1} + s_t * B_t
//   y_t = sum_k C_t (x) h_t + (D * s_t, 0, 0, 0)
// With r = p (x) q, dp = dr (x) conj(q) and dq = conj(p) (x) dr. Walking t backwards
// with g_t = dL/dh_t:
//   g_t      = conj(C_t) (x) gy_t + conj(q_{t+1}) (x) g_{t+1}      (g_T = dL/dh_last)
//   dC_t     = gy_t (x) conj(h_t)
//   dq_t     = g_t (x) conj(h_{t-1})
//   dB_t     = s_t * g_t
//   ds_t     = sum_k <g_t, B_t> + D * gy_t.w,   dD += gy_t.w * s_t
//   dh0      = conj(q_0) (x) g_0
// and dq_t is pulled back through the Cayley closed form (see cayley_pullback)
// to d delta_t (summed over k) and to dalpha, dimag (summed over t here, over b
// by the caller).
//
// States are not stored by the forward: it saves fp32 checkpoints of h at the
// end of every chunk of K steps. The backward walks the chunks from last to
// first; for each it reloads the chunk's operands, recomputes the chunk's K
// states from the previous checkpoint into registers (same arithmetic as the
// forward), then runs the adjoint steps above in reverse. One lane owns one
// (b, d, k); a group of G lanes owns a (b, d) and sums d delta and ds over k
// with the same VALU reduction as the forward.
#pragma once

#include "ssm_scan.hpp"

namespace mqc {

// Store one quaternion (converted from fp32) at byte offset voff + soff of a buffer,
// nontemporal (cache policy NT): dB and dC are 2 x 6.4 GB at config 3, read back only by
// the weight-gradient GEMMs after the whole launch; measured 5.98 -> 5.86 ms there. (The
// same hint on every load made the kernel 23 % slower; on the loads of B and C alone it
// helps, see load_chunk.)
template <typename T>
__device__ inline void store_quat_buf(__amdgpu_buffer_rsrc_t rs, uint32_t voff, const float (&e)[4],
                                      uint32_t soff) {
  constexpr int kNT = 2;  // gfx950 buffer cache-policy bit NT
  if constexpr (sizeof(T) == 4) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = {__float_as_uint(e[0]), __float_as_uint(e[1]), __float_as_uint(e[2]),
                     __float_as_uint(e[3])};
    __builtin_amdgcn_raw_buffer_store_b128(v, rs, voff, soff, kNT);
  } else {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = {pack2<T>(e[0], e[1]), pack2<T>(e[2], e[3])};
    __builtin_amdgcn_raw_buffer_store_b64(v, rs, voff, soff, kNT);
  }
}

struct SsmBwdArgs {
  const void* delta;  // [B,T,D] dtype
  const void* s;      // [B,T,D] dtype
  const void* Bm;     // [B,T,D,S,4] dtype
  const void* Cm;     // [B,T,D,S,4] dtype
  const float* lam_alpha;  // [D,S]
  const float* lam_imag;   // [D,S,3]
  const float* dvec;       // [D]
  const float* h0;         // [B,D,S,4] fp32 or null
  const float* h_ckpt;     // [B,nC,D,S,4] fp32
  const void* gy;          // [B,T,D,4] dtype
  const float* dh_last;    // [B,D,S,4] fp32 or null
  float* d_delta;          // [B,T,D] fp32
  float* d_s;              // [B,T,D] fp32
  void* dB;                // [B,T,D,S,4] dtype
  void* dC;                // [B,T,D,S,4] dtype
  float* dalpha_part;      // [B,D,S]
  float* dimag_part;       // [B,D,S,3]
  float* dD_part;          // [B,D]
  float* dh0;              // [B,D,S,4] fp32 or null
  int64_t batch, T, Dm, S;
  float eps;
  // Time-chunked backward (ssm_bwd_chunked_launch): the T axis in n_chunks
  // chunks of chunk_len steps (a multiple of the checkpoint interval; the last
  // may be shorter), one row of blocks per (chunk, batch). The last chunk starts
  // from dh_last, chunk c < n_chunks - 1 from e_chunk[b, n_chunks - 2 - c]
  // (fp32 [B, n_chunks - 1, D, S, 4]: the adjoint flowing into its last step
  // from the chunks after it). The parameter partials then have
  // n_chunks * batch rows (row chunk * batch + b) and only chunk 0 writes dh0.
  int64_t chunk_len = 0;
  int64_t n_chunks = 1;
  const float* e_chunk = nullptr;
};

// Pull dq back through q = Cayley(dl * Lambda) (closed form, see ssm_scan.hpp):
//   N = 1 - dl a + dl^2 n2 (clamped below at eps), P = 1 - dl^2 n2,
//   q0 = P / N,  qv = dl v / N,  n2 = (a^2 + |v|^2) / 4.
// With r = 1 / max(N, eps), cq = dl r, gq = <dq, q> (taken as 0 where the clamp
// engaged: N is then constant, as in the reference's clamp_min) and
// u = dq.w + gq:
//   d dl  = r (<dq_vec, v> + a gq - 2 dl n2 u)
//   d a   = r (dl gq - (dl^2 / 2) a u)      = cq gq - a (cq dl u) / 2
//   d v_i = r (dl dq_i - (dl^2 / 2) v_i u)  = cq dq_i - v_i (cq dl u) / 2
// The terms that do not involve a or v are summed over t in PullAcc and
// combined with a and v once, after the walk (pull_finish).
struct PullAcc {
  float da = 0.f, dv[3] = {0.f, 0.f, 0.f}, sx = 0.f;
};

// LIVE: the clamp is known not to have engaged (live is then ignored).
template <bool LIVE>
__device__ inline float cayley_pullback(const quat& g, float qw, float cq, float dl, float r,
                                        bool live, const LamConst& L, PullAcc& acc) {
  const float gv = g.x * L.v0 + g.y * L.v1 + g.z * L.v2;  // <dq_vec, v>
  float gq = fmaf(g.w, qw, cq * gv);                        // <dq, q>
  if constexpr (!LIVE) gq = live ? gq : 0.f;
  const float u = g.w + gq;
  const float ddl = fmaf(dl * (-2.f * L.n2), u, fmaf(L.a, gq, gv)) * r;
  acc.sx = fmaf(cq * dl, u, acc.sx);
  acc.da = fmaf(cq, gq, acc.da);
  acc.dv[0] = fmaf(cq, g.x, acc.dv[0]);
  acc.dv[1] = fmaf(cq, g.y, acc.dv[1]);
  acc.dv[2] = fmaf(cq, g.z, acc.dv[2]);
  return ddl;
}

// The gradients w.r.t. a and v from the sums of cayley_pullback.
__device__ inline void pull_finish(const PullAcc& acc, const LamConst& L, float& da, float (&dv)[3]) {
  const float hs = 0.5f * acc.sx;
  da = fmaf(-L.a, hs, acc.da);
  dv[0] = fmaf(-L.v0, hs, acc.dv[0]);
  dv[1] = fmaf(-L.v1, hs, acc.dv[1]);
  dv[2] = fmaf(-L.v2, hs, acc.dv[2]);
}

__device__ inline quat qconj(const quat& q) { return quat{q.w, -q.x, -q.y, -q.z}; }

__device__ inline void qacc(quat& a, const quat& b) {
  a.w += b.w; a.x += b.x; a.y += b.y; a.z += b.z;
}

// Sum two scalars over the G lanes of a group. Afterwards the group's lane 0
// holds the total of u and lane 1 the total of w (G >= 2); for G == 1 the one
// lane holds both (u in u, w in w).
template <int G>
__device__ inline void group_reduce2(float& u, float& w, int lane) {
  if constexpr (G == 1) {
    return;
  } else {
    const bool odd = lane & 1;
    float keep = odd ? w : u;
    const float snd = odd ? u : w;
    keep += lane_xor1(snd);
    if constexpr (G >= 4) keep += lane_xor2(keep);
    if constexpr (G == 8) keep += __shfl_xor(keep, 4);
    if constexpr (G >= 16) {
      keep += row_rot4(keep);
      keep += row_rot8(keep);
    }
    if constexpr (G >= 32) keep = sum_row_pair_to_even(keep);
    if constexpr (G == 64) keep = sum_halves_to_low(keep);
    u = keep;
    w = keep;
  }
}

// SYNC: a block barrier after every chunk keeps the block's waves on the same
// chunk. Unlike the forward, the backward gains nothing from it: about half of
// its traffic is writes (dB, dC), and it moves its bytes at about the rate of a
// plain device copy (4.6-4.7 TB/s at config 3, where a 1 GiB copy runs at
// 4.7-5.3), so the launcher runs free 256-thread blocks, measured 4 % faster
// than lockstep 768-thread ones. Its VALU work (about 160 instructions per step
// and lane at 16-bit storage and G = 64) takes about 3.5 ms of the 5.9.
// Double-buffering the chunk operands was measured too and gave nothing at K = 8.
// WPE caps the registers at two waves per SIMD (<= 256 VGPRs): left alone the
// compiler takes 276 (one wave per SIMD); at three waves per SIMD it spills to
// scratch and runs twice as slow.
template <typename T, int G, int K, int NT, bool FULL, bool SYNC, int WPE = 2>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(WPE))) void ssm_bwd_kernel(SsmBwdArgs a) {
  static_assert((G & (G - 1)) == 0 && G <= 64 && NT % 64 == 0 && NT % G == 0, "bad group");
  constexpr int GPB = NT / G;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int j = tid & (G - 1);
  // Hardware block order. Neighbouring d-blocks share 128-byte lines of delta,
  // s and gy, and the hardware hands them to different XCDs, each of which
  // fetches the line: measured on MI355X (rocprofv3, config 3, bf16) reads at
  // 1.086x the algorithmic bytes in this order against 1.032x with the
  // forward's XCD remap (xcd_block) and 512-thread blocks, whose L2 then holds
  // a whole line. The remap still measured slower (5.92 ms here; 5.99 remapped,
  // 6.34 with 512 threads, 6.14 with both, same buffers): the kernel runs at
  // the box's copy rate, and the 4 % fewer reads do not buy back the order.
  // The write excess (1.024x) is the fp32 d_delta / d_s rows: a block holds 4
  // d's, 16 bytes of each row, which leave the L2 as 12.6 M masked 32-byte
  // writes (TCC_EA0_WRREQ minus TCC_EA0_WRREQ_64B), 0.44 GB for 0.1 GB of data.
  const int64_t by = blockIdx.y;
  const int chunk = a.n_chunks > 1 ? (int)(by / a.batch) : 0;
  const int64_t b = a.n_chunks > 1 ? by - (int64_t)chunk * a.batch : by;
  const int64_t d_raw = (int64_t)blockIdx.x * GPB + tid / G;
  const bool gvalid = d_raw < a.Dm;
  const int64_t d = gvalid ? d_raw : a.Dm - 1;
  const bool kvalid = FULL || j < a.S;
  const int64_t k = kvalid ? j : a.S - 1;
  const bool own = gvalid && kvalid;

  // 32-bit step and chunk counters (the host checks T): gfx9's scalar unit has
  // no 64-bit compares.
  const int Tn = (int)a.T;
  const int nC = (Tn + K - 1) / K;
  const int64_t rowBC = a.Dm * a.S * 4;
  const int64_t rowTok = a.Dm;
  const int64_t rowY = a.Dm * 4;
  const uint32_t offBC = (uint32_t)((d * a.S + k) * 4 * (int64_t)sizeof(T));
  const uint32_t offTok = (uint32_t)(d * (int64_t)sizeof(T));
  const uint32_t offY = (uint32_t)(d * 4 * (int64_t)sizeof(T));
  const int64_t sidx = ((b * a.Dm + d) * a.S + k) * 4;  // this lane's [B,D,S,4] index

  const int64_t dk = d * a.S + k;
  const LamConst L = lam_const(a.lam_alpha, a.lam_imag, dk);
  const float Dv = a.dvec[d];

  PullAcc pacc;
  float dD = 0.f;
  quat carry{0.f, 0.f, 0.f, 0.f};
  if (chunk < a.n_chunks - 1) {
    const int64_t ci = ((b * (a.n_chunks - 1) + (a.n_chunks - 2 - chunk)) * a.Dm + d) * a.S + k;
    float e[4];
    load_vec<float, 4>(a.e_chunk + ci * 4, e);
    carry = quat_from(e);
  } else if (a.dh_last) {
    float e[4];
    load_vec<float, 4>(a.dh_last + sidx, e);
    carry = quat_from(e);
  }

  // Operands of one chunk: the K steps' delta, s, B, C, gy (raw bits) and the
  // checkpointed state before the chunk. Every tensor is read and written
  // through a buffer descriptor on the chunk's first row (SGPRs, rebuilt per
  // chunk); step i adds the scalar i * step bytes and the lane its fixed 32-bit
  // offset, so no addressing runs on the VALU. The launcher checks that K steps
  // of every tensor fit in 32 bits.
  struct Ops {
    Raw<T, 1> rd[K], rs[K];
    Raw<T, 4> rB[K], rC[K], rg[K];
    float4 h_in;
  };
  const uint32_t stepBC = (uint32_t)(rowBC * (int64_t)sizeof(T));
  const uint32_t stepTok = (uint32_t)(rowTok * (int64_t)sizeof(T));
  const uint32_t stepY = (uint32_t)(rowY * (int64_t)sizeof(T));
  const uint32_t stepF = (uint32_t)(rowTok * 4);  // fp32 d_delta, d_s
  const uint32_t offF = (uint32_t)(d * 4);
  auto load_chunk = [&](Ops& o, int c, int len) {
    const int64_t row0 = b * Tn + (int64_t)c * K;
    const __amdgpu_buffer_rsrc_t rD = buf_rsrc((const char*)a.delta + row0 * stepTok);
    const __amdgpu_buffer_rsrc_t rS = buf_rsrc((const char*)a.s + row0 * stepTok);
    const __amdgpu_buffer_rsrc_t rB = buf_rsrc((const char*)a.Bm + row0 * (int64_t)stepBC);
    const __amdgpu_buffer_rsrc_t rC = buf_rsrc((const char*)a.Cm + row0 * (int64_t)stepBC);
    const __amdgpu_buffer_rsrc_t rG = buf_rsrc((const char*)a.gy + row0 * (int64_t)stepY);
#pragma unroll
    for (int i = 0; i < K; ++i) {
      // A tail chunk re-reads its last step.
      const uint32_t ii = (uint32_t)(i < len ? i : len - 1);
      raw_load_buf<T, 1>(rD, offTok, o.rd[i], ii * stepTok);
      raw_load_buf<T, 1>(rS, offTok, o.rs[i], ii * stepTok);
      // B and C with the NT cache policy: each instruction reads whole lines
      // (64 lanes x 8 bytes, or 16 for fp32), read once (5.81-5.84 -> 5.73-5.79 ms
      // at config 4, same buffers). On delta, s and gy, whose lines neighbouring
      // d-blocks share, NT made the kernel 23 % slower.
      raw_load_buf<T, 4, 2>(rB, offBC, o.rB[i], ii * stepBC);
      raw_load_buf<T, 4, 2>(rC, offBC, o.rC[i], ii * stepBC);
      raw_load_buf<T, 4>(rG, offY, o.rg[i], ii * stepY);
    }
    // The checkpoint of the previous chunk (chunk 0 starts from h0, read in process).
    const int64_t cp = c > 0 ? c - 1 : 0;
    o.h_in = *reinterpret_cast<const float4*>(a.h_ckpt + (((b * nC + cp) * a.Dm + d) * a.S + k) * 4);
  };
  // FULLC: all K steps of the chunk exist (every chunk but a ragged last one).
  auto process_chunk = [&](auto fullc, Ops& o, int c, int len) {
    constexpr bool FULLC = decltype(fullc)::value;
    const int64_t row0 = b * Tn + (int64_t)c * K;
    const __amdgpu_buffer_rsrc_t rdB = buf_rsrc((char*)a.dB + row0 * (int64_t)stepBC);
    const __amdgpu_buffer_rsrc_t rdC = buf_rsrc((char*)a.dC + row0 * (int64_t)stepBC);
    const __amdgpu_buffer_rsrc_t rdd = buf_rsrc((char*)a.d_delta + row0 * (int64_t)stepF);
    const __amdgpu_buffer_rsrc_t rds = buf_rsrc((char*)a.d_s + row0 * (int64_t)stepF);
    quat hs[K + 1];
    float rq[K];  // 1 / max(N, eps) of each step
    if (c > 0) {
      hs[0] = quat{o.h_in.x, o.h_in.y, o.h_in.z, o.h_in.w};
    } else if (a.h0) {
      float e[4];
      load_vec<float, 4>(a.h0 + sidx, e);
      hs[0] = quat_from(e);
    } else {
      hs[0] = quat{0.f, 0.f, 0.f, 0.f};
    }
    // Recompute the chunk's states (the forward's arithmetic). `clamped` marks
    // the wave's lanes in which the eps clamp engaged at some step (wave-uniform).
    uint64_t clamped = 0;
#pragma unroll
    for (int i = 0; i < K; ++i) {
      if (FULLC || i < len) {
        const float dl = raw_get(o.rd[i], 0);
        const float dl2 = dl * dl;
        const float Nraw = fmaf(dl2, L.n2, fmaf(-dl, L.a, 1.f));
        const float r = __builtin_amdgcn_rcpf(fmaxf(Nraw, a.eps));
        rq[i] = r;
        clamped |= __builtin_amdgcn_ballot_w64(!(Nraw > a.eps));
        const float cq = dl * r;
        const quat q{fmaf(-dl2, L.n2, 1.f) * r, cq * L.v0, cq * L.v1, cq * L.v2};
        hs[i + 1] = state_step(q, hs[i], raw_get(o.rs[i], 0), raw_quat(o.rB[i], 0));
      }
    }
    // Adjoint steps, last to first. LIVE: no lane of the wave hit the clamp in
    // this chunk (the usual case: in the block N >= 1, as delta >= 0 and a < 0).
    auto adjoint = [&](auto all_live) {
      constexpr bool LIVE = decltype(all_live)::value;
#pragma unroll
      for (int i = K - 1; i >= 0; --i) {
        if (FULLC || i < len) {
          const float dl = raw_get(o.rd[i], 0);
          const float dl2 = dl * dl;
          const float sv = raw_get(o.rs[i], 0);
          const float r = rq[i];
          const float cq = dl * r;
          const float qw = fmaf(-dl2, L.n2, 1.f) * r;
          const quat q{qw, cq * L.v0, cq * L.v1, cq * L.v2};
          bool live = true;
          if constexpr (!LIVE) live = fmaf(dl2, L.n2, fmaf(-dl, L.a, 1.f)) > a.eps;
          const quat gy = raw_quat(o.rg[i], 0);
          const quat Ck = raw_quat(o.rC[i], 0);
          const quat Bk = raw_quat(o.rB[i], 0);
          quat g = carry;
          qmul_acc(g, qconj(Ck), gy);
          quat dq{0.f, 0.f, 0.f, 0.f};
          qmul_acc(dq, g, qconj(hs[i]));
          quat dC{0.f, 0.f, 0.f, 0.f};
          qmul_acc(dC, gy, qconj(hs[i + 1]));
          float ddl = cayley_pullback<LIVE>(dq, qw, cq, dl, r, live, L, pacc);
          float dsk = g.w * Bk.w + g.x * Bk.x + g.y * Bk.y + g.z * Bk.z;
          carry = quat{0.f, 0.f, 0.f, 0.f};
          qmul_acc(carry, qconj(q), g);
          if (own) {
            const float eB[4] = {sv * g.w, sv * g.x, sv * g.y, sv * g.z};
            const float eC[4] = {dC.w, dC.x, dC.y, dC.z};
            store_quat_buf<T>(rdB, offBC, eB, (uint32_t)i * stepBC);
            store_quat_buf<T>(rdC, offBC, eC, (uint32_t)i * stepBC);
          } else {
            ddl = 0.f;
            dsk = 0.f;
          }
          group_reduce2<G>(ddl, dsk, lane);
          // Lane 0 holds the d delta total and lane 1 the ds total; one DPP read
          // brings the latter to lane 0, which stores both. (Stores from two
          // lanes under different conditions get merged by the compiler into
          // one store whose buffer descriptor is lane-dependent, which costs a
          // waterfall loop.)
          const float ds_tot = G > 1 ? lane_xor1(dsk) : dsk;
          if (gvalid && j == 0) {
            store_elem_buf<float>(rdd, offF, ddl, (uint32_t)i * stepF);
            store_elem_buf<float>(rds, offF, fmaf(Dv, gy.w, ds_tot), (uint32_t)i * stepF);
            dD = fmaf(gy.w, sv, dD);
          }
        }
      }
    };
    if (clamped == 0)
      adjoint(std::true_type{});
    else
      adjoint(std::false_type{});
    if constexpr (SYNC) __syncthreads();
  };

  // This block's checkpoint chunks: [c_lo, c_end) (all of them unchunked).
  const int Lc = a.n_chunks > 1 ? (int)a.chunk_len : Tn;
  const int c_lo = a.n_chunks > 1 ? chunk * (Lc / K) : 0;
  const int c_end = chunk == a.n_chunks - 1 ? nC : (chunk + 1) * (Lc / K);
  Ops buf;
  if (c_end > c_lo) {
    const int c = c_end - 1;
    const int len = (int)(Tn - c * K) < K ? (int)(Tn - c * K) : K;
    load_chunk(buf, c, len);
    if (len == K)
      process_chunk(std::integral_constant<bool, true>{}, buf, c, len);
    else
      process_chunk(std::integral_constant<bool, false>{}, buf, c, len);
  }
  for (int c = c_end - 2; c >= c_lo; --c) {
    load_chunk(buf, c, K);
    process_chunk(std::integral_constant<bool, true>{}, buf, c, K);
  }

  const int64_t prow = (int64_t)chunk * a.batch + b;  // partials row
  if (own) {
    if (a.dh0 && chunk == 0) {
      const float e[4] = {carry.w, carry.x, carry.y, carry.z};
      store_vec<float, 4>(a.dh0 + sidx, e);
    }
    float da, dv[3];
    pull_finish(pacc, L, da, dv);
    // Chain to the raw parameters: a = -softplus(alpha), v = tanh(imag).
    const float alpha = a.lam_alpha[dk];
    const float sig = alpha > 20.f ? 1.f : 1.f / (1.f + expf(-alpha));
    a.dalpha_part[prow * a.Dm * a.S + dk] = -da * sig;
    float* di = a.dimag_part + (prow * a.Dm * a.S + dk) * 3;
    di[0] = dv[0] * (1.f - L.v0 * L.v0);
    di[1] = dv[1] * (1.f - L.v1 * L.v1);
    di[2] = dv[2] * (1.f - L.v2 * L.v2);
  }
  if (gvalid && j == 0) a.dD_part[prow * a.Dm + d] = dD;
}

// Checkpoint interval the backward needs: the chunk's operands and states live
// in registers, K steps at a time.
template <typename T>
constexpr int ssm_bwd_chunk() { return sizeof(T) == 4 ? 4 : 8; }

template <typename T, int G>
int launch_ssm_bwd_g(const SsmBwdArgs& a, hipStream_t s) {
  constexpr int K = ssm_bwd_chunk<T>();
  constexpr int NT = 256;
  constexpr int GPB = NT / G;
  const int64_t gx = (a.Dm + GPB - 1) / GPB;
  const int64_t gy = a.batch * a.n_chunks;  // (chunk, batch) rows
  if (gx > 0x7fffffffLL || gy > 65535) return MQC_E_LIMIT;
  const dim3 grid((unsigned)gx, (unsigned)gy);
  if (a.S == G)
    ssm_bwd_kernel<T, G, K, NT, true, false><<<grid, dim3(NT), 0, s>>>(a);
  else
    ssm_bwd_kernel<T, G, K, NT, false, false><<<grid, dim3(NT), 0, s>>>(a);
  return launch_status();
}

// What every launch of the backward needs of its arguments, checked on the
// host before any kernel runs (the chunked backward calls it before its carry
// launch).
template <typename T>
int ssm_bwd_check(const SsmBwdArgs& a) {
  // K consecutive steps of one tensor must be addressable with 32-bit offsets.
  if (a.Dm * a.S * 4 * (int64_t)sizeof(T) * ssm_bwd_chunk<T>() >= ((int64_t)1 << 32))
    return MQC_E_LIMIT;
  if (a.T >= ((int64_t)1 << 30)) return MQC_E_LIMIT;
  const uintptr_t qa = 4 * sizeof(T);
  if (!aligned(a.Bm, qa) || !aligned(a.Cm, qa) || !aligned(a.gy, qa) || !aligned(a.dB, qa) ||
      !aligned(a.dC, qa) || !aligned(a.h_ckpt, 16) || (a.h0 && !aligned(a.h0, 16)) ||
      (a.dh_last && !aligned(a.dh_last, 16)) || (a.dh0 && !aligned(a.dh0, 16)) ||
      !aligned(a.delta, sizeof(T)) || !aligned(a.s, sizeof(T)) || !aligned(a.d_delta, 4) ||
      !aligned(a.d_s, 4))
    return MQC_E_ALIGN;
  return MQC_OK;
}

template <typename T>
int launch_ssm_bwd(const SsmBwdArgs& a, hipStream_t s) {
  // T == 0 still launches: the walk is empty, dh0 = dh_last and the parameter
  // partials are zero.
  if (a.batch == 0 || a.Dm == 0) return MQC_OK;
  const int chk = ssm_bwd_check<T>(a);
  if (chk != MQC_OK) return chk;
  const int64_t S = a.S;
  if (S <= 1) return launch_ssm_bwd_g<T, 1>(a, s);
  if (S <= 2) return launch_ssm_bwd_g<T, 2>(a, s);
  if (S <= 4) return launch_ssm_bwd_g<T, 4>(a, s);
  if (S <= 8) return launch_ssm_bwd_g<T, 8>(a, s);
  if (S <= 16) return launch_ssm_bwd_g<T, 16>(a, s);
  if (S <= 32) return launch_ssm_bwd_g<T, 32>(a, s);
  if (S <= 64) return launch_ssm_bwd_g<T, 64>(a, s);
  return MQC_E_LIMIT;
}

extern template int launch_ssm_bwd<float>(const SsmBwdArgs&, hipStream_t);
extern template int launch_ssm_bwd<bf16_t>(const SsmBwdArgs&, hipStream_t);
extern template int launch_ssm_bwd<f16_t>(const SsmBwdArgs&, hipStream_t);

}  // namespace mqc
