// C ABI of the fused quaternion SSM's training forward (state checkpoints) and
// backward (kernels: ssm_scan.hpp, ssm_bwd.hpp), whole or time-chunked
// (ssm_chunk.hpp, ssm_bwd_chunk.hpp).
#include "ssm_bwd_chunk.hpp"

using namespace mqc;

extern "C" {

int mqc_ssm_bwd_ckpt_every(int dtype) {
  switch (dtype) {
    case MQC_F32: return ssm_bwd_chunk<float>();
    case MQC_BF16: return ssm_bwd_chunk<bf16_t>();
    case MQC_F16: return ssm_bwd_chunk<f16_t>();
    default: return MQC_E_DTYPE;
  }
}

int mqc_ssm_fused_fwd_train(const void* delta, const void* s, const void* B, const void* C,
                            const float* lambda_alpha, const float* lambda_imag, const float* D,
                            const void* h0, void* y, void* h_last, float* h_ckpt,
                            int64_t ckpt_every, int64_t batch, int64_t seq_len, int64_t d_inner,
                            int64_t d_state, float eps, int dtype, void* stream) {
  if (batch < 0 || seq_len < 0 || d_inner < 0 || d_state < 0 || ckpt_every < 1)
    return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  // An empty walk (seq_len 0) still writes h_last: h0, or zeros without h0.
  const bool steps = batch > 0 && d_inner > 0 && seq_len > 0;
  const bool state_only = batch > 0 && d_inner > 0 && seq_len == 0 && h_last && d_state > 0;
  if (steps && d_state == 0) return MQC_E_SHAPE;
  if (steps && (!delta || !s || !B || !C || !y || !h_ckpt)) return MQC_E_NULL;
  if ((steps || state_only) && (!lambda_alpha || !lambda_imag || !D)) return MQC_E_NULL;
  if (batch > 65535 || d_inner > (1LL << 24) || d_state > 256) return MQC_E_LIMIT;
  if (h_ckpt && !aligned(h_ckpt, 16)) return MQC_E_ALIGN;
  SsmArgs a{};
  a.delta = delta; a.s = s; a.lam_alpha = lambda_alpha; a.lam_imag = lambda_imag; a.dvec = D;
  a.Bm = B; a.Cm = C; a.h0 = h0; a.y = y; a.h_last = h_last;
  a.h_ckpt = steps ? h_ckpt : nullptr; a.ckpt_every = ckpt_every;
  a.batch = batch; a.T = seq_len; a.Dm = d_inner; a.S = d_state; a.eps = eps;
  if (!steps && !state_only) return MQC_OK;
  switch (dtype) {
    case MQC_F32: return launch_ssm<float, MODE_DL>(a, (hipStream_t)stream);
    case MQC_BF16: return launch_ssm<bf16_t, MODE_DL>(a, (hipStream_t)stream);
    default: return launch_ssm<f16_t, MODE_DL>(a, (hipStream_t)stream);
  }
}

int mqc_ssm_fused_bwd(const void* delta, const void* s, const void* B, const void* C,
                      const float* lambda_alpha, const float* lambda_imag, const float* D,
                      const void* h0, const float* h_ckpt, int64_t ckpt_every, const void* gy,
                      const void* dh_last, float* d_delta, float* d_s, void* dB, void* dC,
                      float* dlambda_alpha_part, float* dlambda_imag_part, float* dD_part,
                      void* dh0, int64_t batch, int64_t seq_len, int64_t d_inner,
                      int64_t d_state, float eps, int dtype, void* stream) {
  if (batch < 0 || seq_len < 0 || d_inner < 0 || d_state < 0) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  // An empty walk (seq_len 0) still writes its outputs: dh0 = dh_last (zeros
  // without it) and zero parameter partials.
  const bool steps = batch > 0 && d_inner > 0 && seq_len > 0;
  const bool empty_walk = batch > 0 && d_inner > 0 && seq_len == 0 && d_state > 0;
  if (steps && d_state == 0) return MQC_E_SHAPE;
  if (steps && (!delta || !s || !B || !C || !h_ckpt || !gy || !d_delta || !d_s || !dB || !dC))
    return MQC_E_NULL;
  if ((steps || empty_walk) && (!lambda_alpha || !lambda_imag || !D || !dlambda_alpha_part ||
                                !dlambda_imag_part || !dD_part))
    return MQC_E_NULL;
  if (batch > 65535 || d_inner > (1LL << 24) || d_state > 64) return MQC_E_LIMIT;
  if (ckpt_every != mqc_ssm_bwd_ckpt_every(dtype)) return MQC_E_LIMIT;
  SsmBwdArgs a{};
  a.delta = delta; a.s = s; a.Bm = B; a.Cm = C; a.lam_alpha = lambda_alpha;
  a.lam_imag = lambda_imag; a.dvec = D; a.h0 = (const float*)h0; a.h_ckpt = h_ckpt; a.gy = gy;
  a.dh_last = (const float*)dh_last; a.d_delta = d_delta; a.d_s = d_s; a.dB = dB; a.dC = dC;
  a.dalpha_part = dlambda_alpha_part; a.dimag_part = dlambda_imag_part; a.dD_part = dD_part;
  a.dh0 = (float*)dh0; a.batch = batch; a.T = seq_len; a.Dm = d_inner; a.S = d_state; a.eps = eps;
  if (!steps && !empty_walk) return MQC_OK;
  switch (dtype) {
    case MQC_F32: return launch_ssm_bwd<float>(a, (hipStream_t)stream);
    case MQC_BF16: return launch_ssm_bwd<bf16_t>(a, (hipStream_t)stream);
    default: return launch_ssm_bwd<f16_t>(a, (hipStream_t)stream);
  }
}

namespace {

// What the chunked entry points add to the whole ones' checks: the chunk
// length (a multiple of the checkpoint interval), the workspace and the
// chunked launches' limits. Sets n_chunks (1: run the whole walk).
int check_chunk_args(int64_t batch, int64_t seq_len, int64_t d_inner, int64_t d_state,
                     int64_t chunk_len, int64_t ckpt_every, const void* workspace,
                     int64_t workspace_bytes, int64_t& n_chunks) {
  n_chunks = 1;
  if (chunk_len < 1 || ckpt_every < 1 || chunk_len % ckpt_every != 0) return MQC_E_SHAPE;
  if (seq_len <= chunk_len || batch == 0 || d_inner == 0) return MQC_OK;
  if (d_state > kChunkMaxState) return MQC_E_LIMIT;
  n_chunks = (seq_len + chunk_len - 1) / chunk_len;
  if (batch * n_chunks > 65535) return MQC_E_LIMIT;
  if (workspace_bytes < ssm_chunk_workspace_bytes(batch, seq_len, d_inner, d_state, chunk_len))
    return MQC_E_SPACE;
  if (!workspace) return MQC_E_NULL;
  if (!aligned(workspace, 16)) return MQC_E_ALIGN;
  return MQC_OK;
}

}  // namespace

int mqc_ssm_fused_fwd_train_chunked(const void* delta, const void* s, const void* B,
                                    const void* C, const float* lambda_alpha,
                                    const float* lambda_imag, const float* D, const void* h0,
                                    void* y, void* h_last, float* h_ckpt, int64_t ckpt_every,
                                    int64_t batch, int64_t seq_len, int64_t d_inner,
                                    int64_t d_state, int64_t chunk_len, float eps, int dtype,
                                    void* workspace, int64_t workspace_bytes, void* stream) {
  if (batch < 0 || seq_len < 0 || d_inner < 0 || d_state < 0) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  int64_t nc = 1;
  const int st = check_chunk_args(batch, seq_len, d_inner, d_state, chunk_len, ckpt_every,
                                  workspace, workspace_bytes, nc);
  if (st != MQC_OK) return st;
  if (nc <= 1)
    return mqc_ssm_fused_fwd_train(delta, s, B, C, lambda_alpha, lambda_imag, D, h0, y, h_last,
                                   h_ckpt, ckpt_every, batch, seq_len, d_inner, d_state, eps,
                                   dtype, stream);
  if (d_state == 0) return MQC_E_SHAPE;
  if (!delta || !s || !B || !C || !y || !h_ckpt || !lambda_alpha || !lambda_imag || !D)
    return MQC_E_NULL;
  if (d_inner > (1LL << 24)) return MQC_E_LIMIT;
  if (!aligned(h_ckpt, 16)) return MQC_E_ALIGN;
  // As in mqc_ssm_fused_fwd_chunked: chunk 0 reads h0, the last chunk writes
  // h_last, in one launch.
  const int64_t state_bytes = batch * d_inner * d_state * 4 * (int64_t)sizeof(float);
  if (overlaps(h0, state_bytes, h_last, state_bytes)) return MQC_E_OVERLAP;
  SsmArgs a{};
  a.delta = delta; a.s = s; a.lam_alpha = lambda_alpha; a.lam_imag = lambda_imag; a.dvec = D;
  a.Bm = B; a.Cm = C; a.h0 = h0; a.y = y; a.h_last = h_last;
  a.h_ckpt = h_ckpt; a.ckpt_every = ckpt_every;
  a.batch = batch; a.T = seq_len; a.Dm = d_inner; a.S = d_state; a.eps = eps;
  a.chunk_len = chunk_len; a.n_chunks = nc;
  switch (dtype) {
    case MQC_F32: return ssm_chunk_launch<float>(a, (float*)workspace, (hipStream_t)stream);
    case MQC_BF16: return ssm_chunk_launch<bf16_t>(a, (float*)workspace, (hipStream_t)stream);
    default: return ssm_chunk_launch<f16_t>(a, (float*)workspace, (hipStream_t)stream);
  }
}

int mqc_ssm_fused_bwd_chunked(const void* delta, const void* s, const void* B, const void* C,
                              const float* lambda_alpha, const float* lambda_imag, const float* D,
                              const void* h0, const float* h_ckpt, int64_t ckpt_every,
                              const void* gy, const void* dh_last, float* d_delta, float* d_s,
                              void* dB, void* dC, float* dlambda_alpha_part,
                              float* dlambda_imag_part, float* dD_part, void* dh0, int64_t batch,
                              int64_t seq_len, int64_t d_inner, int64_t d_state,
                              int64_t chunk_len, float eps, int dtype, void* workspace,
                              int64_t workspace_bytes, void* stream) {
  if (batch < 0 || seq_len < 0 || d_inner < 0 || d_state < 0) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  int64_t nc = 1;
  const int st = check_chunk_args(batch, seq_len, d_inner, d_state, chunk_len, ckpt_every,
                                  workspace, workspace_bytes, nc);
  if (st != MQC_OK) return st;
  if (nc <= 1)
    return mqc_ssm_fused_bwd(delta, s, B, C, lambda_alpha, lambda_imag, D, h0, h_ckpt,
                             ckpt_every, gy, dh_last, d_delta, d_s, dB, dC, dlambda_alpha_part,
                             dlambda_imag_part, dD_part, dh0, batch, seq_len, d_inner, d_state,
                             eps, dtype, stream);
  if (d_state == 0) return MQC_E_SHAPE;
  if (!delta || !s || !B || !C || !h_ckpt || !gy || !d_delta || !d_s || !dB || !dC ||
      !lambda_alpha || !lambda_imag || !D || !dlambda_alpha_part || !dlambda_imag_part ||
      !dD_part)
    return MQC_E_NULL;
  if (d_inner > (1LL << 24) || d_state > 64) return MQC_E_LIMIT;
  if (ckpt_every != mqc_ssm_bwd_ckpt_every(dtype)) return MQC_E_LIMIT;
  // The last chunk reads dh_last as it starts and chunk 0 writes dh0 as it
  // ends, in one launch.
  const int64_t state_bytes = batch * d_inner * d_state * 4 * (int64_t)sizeof(float);
  if (overlaps(dh_last, state_bytes, dh0, state_bytes)) return MQC_E_OVERLAP;
  SsmBwdArgs a{};
  a.delta = delta; a.s = s; a.Bm = B; a.Cm = C; a.lam_alpha = lambda_alpha;
  a.lam_imag = lambda_imag; a.dvec = D; a.h0 = (const float*)h0; a.h_ckpt = h_ckpt; a.gy = gy;
  a.dh_last = (const float*)dh_last; a.d_delta = d_delta; a.d_s = d_s; a.dB = dB; a.dC = dC;
  a.dalpha_part = dlambda_alpha_part; a.dimag_part = dlambda_imag_part; a.dD_part = dD_part;
  a.dh0 = (float*)dh0; a.batch = batch; a.T = seq_len; a.Dm = d_inner; a.S = d_state; a.eps = eps;
  a.chunk_len = chunk_len; a.n_chunks = nc;
  switch (dtype) {
    case MQC_F32: return ssm_bwd_chunked_launch<float>(a, (float*)workspace, (hipStream_t)stream);
    case MQC_BF16: return ssm_bwd_chunked_launch<bf16_t>(a, (float*)workspace, (hipStream_t)stream);
    default: return ssm_bwd_chunked_launch<f16_t>(a, (float*)workspace, (hipStream_t)stream);
  }
}

}  // extern "C"
