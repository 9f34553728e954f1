// C ABI of the fused quaternion SSM (kernels and launch shapes: ssm_scan.hpp).
#include "ssm_scan.hpp"

namespace mqc {

template <int MODE>
int dispatch_ssm(const SsmArgs& a, int dtype, hipStream_t s) {
  switch (dtype) {
    case MQC_F32: return launch_ssm<float, MODE>(a, s);
    case MQC_BF16: return launch_ssm<bf16_t, MODE>(a, s);
    case MQC_F16: return launch_ssm<f16_t, MODE>(a, s);
    default: return MQC_E_DTYPE;
  }
}

}  // namespace mqc

using namespace mqc;

extern "C" {

int mqc_ssm_q_fwd(const void* q, const void* B, const void* S, const void* C, const void* D,
                  int64_t d_sb, int64_t d_st, int64_t d_sd, const void* h0, void* y,
                  void* h_last, int64_t batch, int64_t seq_len, int64_t d_inner,
                  int64_t d_state, int dtype, void* stream) {
  if (batch < 0 || seq_len < 0 || d_inner < 0 || d_state < 0) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  // An empty walk (seq_len 0) still writes h_last: h0, or zeros without h0.
  const bool steps = batch > 0 && d_inner > 0 && seq_len > 0;
  const bool state_only = batch > 0 && d_inner > 0 && seq_len == 0 && h_last && d_state > 0;
  if (steps && d_state == 0) return MQC_E_SHAPE;
  if (steps && (!q || !B || !S || !C || !D || !y)) return MQC_E_NULL;
  if (batch > 65535 || d_inner > (1LL << 24) || d_state > 256) return MQC_E_LIMIT;
  const int64_t elsize = dtype == MQC_F32 ? 4 : 2;
  if (partial_overlap(h0, h_last, batch * d_inner * d_state * 4 * elsize)) return MQC_E_OVERLAP;
  SsmArgs a{};
  a.q = q; a.Sq = S; a.Dq = D; a.d_sb = d_sb; a.d_st = d_st; a.d_sd = d_sd;
  a.Bm = B; a.Cm = C; a.h0 = h0; a.y = y; a.h_last = h_last;
  a.batch = batch; a.T = seq_len; a.Dm = d_inner; a.S = d_state; a.eps = 0.f;
  if (!steps && !state_only) return MQC_OK;
  return dispatch_ssm<MODE_Q>(a, dtype, (hipStream_t)stream);
}

int mqc_ssm_fused_fwd(const void* delta, const void* s, const void* B, const void* C,
                      const float* lambda_alpha, const float* lambda_imag, const float* D,
                      const void* h0, void* y, void* h_last, int64_t batch, int64_t seq_len,
                      int64_t d_inner, int64_t d_state, float eps, int dtype, void* stream) {
  if (batch < 0 || seq_len < 0 || d_inner < 0 || d_state < 0) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  // An empty walk (seq_len 0) still writes h_last: h0, or zeros without h0.
  const bool steps = batch > 0 && d_inner > 0 && seq_len > 0;
  const bool state_only = batch > 0 && d_inner > 0 && seq_len == 0 && h_last && d_state > 0;
  if (steps && d_state == 0) return MQC_E_SHAPE;
  if (steps && (!delta || !s || !B || !C || !y)) return MQC_E_NULL;
  if ((steps || state_only) && (!lambda_alpha || !lambda_imag || !D)) return MQC_E_NULL;
  if (batch > 65535 || d_inner > (1LL << 24) || d_state > 256) return MQC_E_LIMIT;
  if (partial_overlap(h0, h_last, batch * d_inner * d_state * 4 * (int64_t)sizeof(float)))
    return MQC_E_OVERLAP;
  SsmArgs a{};
  a.delta = delta; a.s = s; a.lam_alpha = lambda_alpha; a.lam_imag = lambda_imag; a.dvec = D;
  a.Bm = B; a.Cm = C; a.h0 = h0; a.y = y; a.h_last = h_last;
  a.batch = batch; a.T = seq_len; a.Dm = d_inner; a.S = d_state; a.eps = eps;
  if (!steps && !state_only) return MQC_OK;
  return dispatch_ssm<MODE_DL>(a, dtype, (hipStream_t)stream);
}

}  // extern "C"
