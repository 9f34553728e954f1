#pragma once
// Time-chunked backward of the block's fused quaternion SSM.
//
// The backward (ssm_bwd.hpp) walks each (b, d, k) lane from the last step to
// the first, carrying the adjoint e (the gradient reaching step t from the
// steps after it):
//   g_t = e_t + conj(C_t) (x) gy_t,      e_{t-1} = conj(q_t) (x) g_t,
// with e at the last step = dL/dh_last. Over a chunk of steps [t0, t1) the
// adjoint leaving its first step is an affine map of the one entering its last:
//   e_out = P (x) e_in + H,   P = conj(q_t0) (x) ... (x) conj(q_t1-1),
// H = e_out from e_in = 0. Every q of a lane is qw + c v with the lane's fixed
// pure v, so P = Pa + Pb v as in the forward's chunked walk (ssm_chunk.hpp),
// and chunks compose the same way, the chunk processed later on the left.
// Laid out in processing order (last chunk first) the maps are exactly what
// the forward's wave-level prefix (ssm_carry_prefix_kernel) scans, with
// dL/dh_last in the place of h0. Three launches:
//   1. ssm_bwd_agg_kernel: every chunk but the first walks its steps backward
//      from e = 0, reading delta, C and gy, and stores (P, H) at row
//      n_chunks - 1 - c of the workspace;
//   2. ssm_carry_prefix_kernel: row r then holds the adjoint entering the last
//      step of chunk n_chunks - 2 - r;
//   3. ssm_bwd_kernel with the chunk fields set: every chunk runs the usual
//      backward from its entering adjoint (the last from dL/dh_last).
// Chunk boundaries fall on checkpoint boundaries (chunk_len is a multiple of
// the checkpoint interval), so launch 3 reads the forward's checkpoints as
// they are. The parameter gradients come out as per-(chunk, batch) partials.
#include "ssm_bwd.hpp"
#include "ssm_chunk.hpp"

namespace mqc {

template <typename T>
struct BwdAggStep {
  Raw<T, 1> delta;
  Raw<T, 4> C, gy;
};

// Launch 1. Grid (d-blocks, batch * (n_chunks - 1)); block row by = r * batch +
// b holds chunk c = n_chunks - 1 - r (r = 0 is the last chunk, the only one
// that may be shorter than chunk_len). One lane per (b, d, k), G lanes per d.
// Hc: fp32 [B, n_chunks - 1, D, S, 4]; Pc: fp32 [B, n_chunks - 1, D, S, 2].
template <typename T, int G, int PF, int NT, bool FULL>
__global__ __launch_bounds__(NT) void ssm_bwd_agg_kernel(SsmBwdArgs a, float* Hc, float* Pc) {
  static_assert((G & (G - 1)) == 0 && G <= 64 && NT % 64 == 0 && NT % G == 0, "bad group");
  constexpr int GPB = NT / G;
  const int tid = threadIdx.x;
  const int j = tid & (G - 1);
  const int64_t by = blockIdx.y;
  const int r = (int)(by / a.batch);
  const int64_t b = by - (int64_t)r * a.batch;
  const int chunk = (int)a.n_chunks - 1 - r;
  const int64_t d_raw = (int64_t)blockIdx.x * GPB + tid / G;
  const bool gvalid = d_raw < a.Dm;
  const int64_t d = gvalid ? d_raw : a.Dm - 1;
  const bool kvalid = FULL || j < a.S;
  const int64_t k = kvalid ? j : a.S - 1;

  const int Tn = (int)a.T;
  const int Lc = (int)a.chunk_len;
  const int t0 = chunk * Lc;
  const int t1 = t0 + Lc < Tn ? t0 + Lc : Tn;
  const int len = t1 - t0;
  const int64_t rowBC = a.Dm * a.S * 4;
  const int64_t rowTok = a.Dm;
  const int64_t rowY = a.Dm * 4;
  const uint32_t offBC = (uint32_t)((d * a.S + k) * 4 * (int64_t)sizeof(T));
  const uint32_t offTok = (uint32_t)(d * (int64_t)sizeof(T));
  const uint32_t offY = (uint32_t)(d * 4 * (int64_t)sizeof(T));

  const int64_t dk = d * a.S + k;
  const LamConst L = lam_const(a.lam_alpha, a.lam_imag, dk);
  const float vv = L.v0 * L.v0 + L.v1 * L.v1 + L.v2 * L.v2;

  auto load_step = [&](BwdAggStep<T>& st, int t) {
    const int64_t rt = b * Tn + t;
    raw_load_buf<T, 1>(buf_rsrc((const T*)a.delta + rt * rowTok), offTok, st.delta);
    raw_load_buf<T, 4>(buf_rsrc((const T*)a.Cm + rt * rowBC), offBC, st.C);
    raw_load_buf<T, 4>(buf_rsrc((const T*)a.gy + rt * rowY), offY, st.gy);
  };
  quat e{0.f, 0.f, 0.f, 0.f};
  float pa = 1.f, pb = 0.f;
  // Step t (walked from t1 - 1 down to t0); refill with the step PF earlier
  // (clamped at t0: the last group re-reads t0, which keeps the loads
  // unconditional).
  auto step = [&](auto refill, BwdAggStep<T>& cur, int t) {
    constexpr bool REFILL = decltype(refill)::value;
    const float dl = raw_get(cur.delta, 0);
    float c;
    const quat q = cayley_step_c(dl, dl * dl, L, a.eps, c);
    quat g = e;
    qmul_acc(g, qconj(raw_quat(cur.C, 0)), raw_quat(cur.gy, 0));
    e = quat{0.f, 0.f, 0.f, 0.f};
    qmul_acc(e, qconj(q), g);
    // P <- conj(q) P with conj(q) = q.w - c v.
    const float na = fmaf(q.w, pa, c * pb * vv);
    pb = fmaf(q.w, pb, -c * pa);
    pa = na;
    if constexpr (REFILL) {
      const int tn = t - PF;
      load_step(cur, tn >= t0 ? tn : t0);
    }
  };

  BwdAggStep<T> ring[PF];
  int i0 = 0;
  if (len >= PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      load_step(ring[i], t1 - 1 - i);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (; i0 + PF <= len; i0 += PF) {
#pragma unroll
      for (int i = 0; i < PF; ++i) step(std::true_type{}, ring[i], t1 - 1 - (i0 + i));
    }
  } else {
#pragma unroll
    for (int i = 0; i < PF; ++i)
      if (i < len) load_step(ring[i], t1 - 1 - i);
  }
  if (i0 < len) {
#pragma unroll
    for (int i = 0; i < PF; ++i)
      if (i0 + i < len) step(std::false_type{}, ring[i], t1 - 1 - (i0 + i));
  }

  if (gvalid && kvalid) {
    const int64_t idx = ((b * (a.n_chunks - 1) + r) * a.Dm + d) * a.S + k;
    const float h4[4] = {e.w, e.x, e.y, e.z};
    store_vec<float, 4>(Hc + idx * 4, h4);
    Pc[idx * 2 + 0] = pa;
    Pc[idx * 2 + 1] = pb;
  }
}

template <typename T, int G>
int launch_bwd_agg_g(const SsmBwdArgs& a, float* Hc, float* Pc, hipStream_t s) {
  constexpr int NT = 256;
  constexpr int PF = 8;
  constexpr int GPB = NT / G;
  const int64_t gx = (a.Dm + GPB - 1) / GPB;
  const int64_t gy = a.batch * (a.n_chunks - 1);
  if (gx > 0x7fffffffLL || gy > 65535) return MQC_E_LIMIT;
  const dim3 grid((unsigned)gx, (unsigned)gy);
  if (a.S == G)
    ssm_bwd_agg_kernel<T, G, PF, NT, true><<<grid, dim3(NT), 0, s>>>(a, Hc, Pc);
  else
    ssm_bwd_agg_kernel<T, G, PF, NT, false><<<grid, dim3(NT), 0, s>>>(a, Hc, Pc);
  return launch_status();
}

// The three launches of the chunked backward. a.chunk_len (a multiple of the
// checkpoint interval) and a.n_chunks (> 1) are set; ws holds
// ssm_chunk_workspace_bytes; the caller has checked the arguments as for the
// whole backward.
template <typename T>
int ssm_bwd_chunked_launch(const SsmBwdArgs& a0, float* ws, hipStream_t s) {
  SsmBwdArgs a = a0;
  // The backward's own argument checks, before the carry launch reads anything.
  const int chk = ssm_bwd_check<T>(a);
  if (chk != MQC_OK) return chk;
  const int64_t nc = a.n_chunks - 1;
  float* Hc = ws;
  float* Pc = ws + a.batch * nc * a.Dm * a.S * 4;
  int st;
  const int64_t S = a.S;
  if (S <= 1) st = launch_bwd_agg_g<T, 1>(a, Hc, Pc, s);
  else if (S <= 2) st = launch_bwd_agg_g<T, 2>(a, Hc, Pc, s);
  else if (S <= 4) st = launch_bwd_agg_g<T, 4>(a, Hc, Pc, s);
  else if (S <= 8) st = launch_bwd_agg_g<T, 8>(a, Hc, Pc, s);
  else if (S <= 16) st = launch_bwd_agg_g<T, 16>(a, Hc, Pc, s);
  else if (S <= 32) st = launch_bwd_agg_g<T, 32>(a, Hc, Pc, s);
  else if (S <= 64) st = launch_bwd_agg_g<T, 64>(a, Hc, Pc, s);
  else return MQC_E_LIMIT;
  if (st != MQC_OK) return st;
  // The forward's prefix over the same layout, dL/dh_last in the place of h0.
  SsmArgs p{};
  p.lam_alpha = a.lam_alpha;
  p.lam_imag = a.lam_imag;
  p.h0 = a.dh_last;
  p.batch = a.batch;
  p.T = a.T;
  p.Dm = a.Dm;
  p.S = a.S;
  p.n_chunks = a.n_chunks;
  p.chunk_len = a.chunk_len;
  if (nc <= 1) st = launch_carry_prefix<1>(p, Hc, Pc, s);
  else if (nc <= 2) st = launch_carry_prefix<2>(p, Hc, Pc, s);
  else if (nc <= 4) st = launch_carry_prefix<4>(p, Hc, Pc, s);
  else if (nc <= 8) st = launch_carry_prefix<8>(p, Hc, Pc, s);
  else if (nc <= 16) st = launch_carry_prefix<16>(p, Hc, Pc, s);
  else if (nc <= 32) st = launch_carry_prefix<32>(p, Hc, Pc, s);
  else st = launch_carry_prefix<64>(p, Hc, Pc, s);
  if (st != MQC_OK) return st;
  a.e_chunk = Hc;
  return launch_ssm_bwd<T>(a, s);
}

extern template int ssm_bwd_chunked_launch<float>(const SsmBwdArgs&, float*, hipStream_t);
extern template int ssm_bwd_chunked_launch<bf16_t>(const SsmBwdArgs&, float*, hipStream_t);
extern template int ssm_bwd_chunked_launch<f16_t>(const SsmBwdArgs&, float*, hipStream_t);

}  // namespace mqc
