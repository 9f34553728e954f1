// C ABI of the time-chunked fused SSM walk (kernels and launches: ssm_chunk.hpp).
#include <mutex>

#include "ssm_chunk.hpp"

using namespace mqc;

// Fixed device scratch of mqc_ssm_fused_fwd_chunked_noalloc: the chunk
// transitions live here instead of in a caller's workspace. Each device the
// library runs on holds its own copy for the life of the process. In host code
// `scratch` names a host-side stand-in, never the device memory: the device
// address comes from hipGetSymbolAddress, once per device (scratch_ptr).
constexpr int64_t kScratchBytes = (int64_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on the first call on
// each device, with that device current).
int scratch_ptr(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return MQC_E_LIMIT;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return (int)hipErrorInvalidSymbol;
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return MQC_OK;
}

// Chunks are at least this long: each chunk pays one extra walk over its
// delta, s and B (the carry launch) and a short prefix launch.
constexpr int64_t kMinChunk = 64;
// The whole walk keeps the machine busy from this many states up (config 3:
// 4 x 1536 x 64); fewer get chunks until states x chunks reaches it, at most
// kMaxChunks. Measured on MI355X (bf16, whole walk -> best chunking, ms):
// T 2048: B1 d_inner 1536 S64 0.964 -> 0.824 (4 chunks), B1 d768 S64
// 0.698 -> 0.426 (8), B1 T4096 d1536 S64 1.82 -> 1.64 (4); B2 d1536 S64 1.25
// and B4 d1536 S16 0.85 only got slower (1.37, 0.90 with 2 chunks): the carry
// launch re-reads B, 25-38 % more bytes, which only pays where the whole walk
// is far from the bandwidth. Long walks of few states (the d-slices of a long
// sequence): B1 T262144 d8 S64 88.4 -> 0.65 (512 chunks; 17.3 with 8),
// B1 T65536 d32 S64 22.8 -> 0.61 (256), B1 T16384 d96 S64 5.70 -> 0.47 (64).
constexpr int64_t kBusyStates = 393216;
constexpr int64_t kMaxChunks = 1024;
// Below 32 states per (b, d) the whole walk already packs one state per lane
// into short groups; chunk those only when the states are fewer than this.
constexpr int64_t kFewStates = 49152;

int64_t auto_chunk_len(int64_t batch, int64_t T, int64_t Dm, int64_t S) {
  if (batch <= 0 || Dm <= 0 || S <= 0 || S > kChunkMaxState || T < 2 * kMinChunk) return T;
  const int64_t states = batch * Dm * S;
  if (states >= kBusyStates / 2 || (S < 32 && states > kFewStates)) return T;
  int64_t nc = (kBusyStates + states - 1) / states;
  if (nc > kMaxChunks) nc = kMaxChunks;
  if (nc > T / kMinChunk) nc = T / kMinChunk;
  // The chunked launches put batch * n_chunks blocks on the grid's y axis.
  if (nc > 65535 / batch) nc = 65535 / batch;
  if (nc <= 1) return T;
  // ceil(T / L) never exceeds nc for L = ceil(T / nc).
  return (T + nc - 1) / nc;
}

// Everything mqc_ssm_fused_fwd checks, plus the chunk length. Returns MQC_OK
// with *nothing set when there is nothing to launch.
int check_chunked(const void* delta, const void* s, const void* B, const void* C,
                  const float* lambda_alpha, const float* lambda_imag, const float* D,
                  const void* h0, const void* y, const void* h_last, int64_t batch,
                  int64_t seq_len, int64_t d_inner, int64_t d_state, int64_t chunk_len,
                  int dtype, bool& nothing) {
  nothing = false;
  if (batch < 0 || seq_len < 0 || d_inner < 0 || d_state < 0 || chunk_len < 1) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  const bool steps = batch > 0 && d_inner > 0 && seq_len > 0;
  const bool state_only = batch > 0 && d_inner > 0 && seq_len == 0 && h_last && d_state > 0;
  if (steps && d_state == 0) return MQC_E_SHAPE;
  if (steps && (!delta || !s || !B || !C || !y)) return MQC_E_NULL;
  if ((steps || state_only) && (!lambda_alpha || !lambda_imag || !D)) return MQC_E_NULL;
  if (batch > 65535 || d_inner > (1LL << 24) || d_state > 256) return MQC_E_LIMIT;
  nothing = !steps && !state_only;
  // With more than one chunk, chunk 0 reads h0 as it starts and the last chunk
  // writes h_last as it ends, in blocks of one launch that run in no fixed
  // order: no in-place state (the whole walk allows it).
  const int64_t state_bytes = batch * d_inner * d_state * 4 * (int64_t)sizeof(float);
  if (steps && seq_len > chunk_len && overlaps(h0, state_bytes, h_last, state_bytes))
    return MQC_E_OVERLAP;
  if (partial_overlap(h0, h_last, state_bytes)) return MQC_E_OVERLAP;
  return MQC_OK;
}

template <typename T>
int run_chunked(SsmArgs& a, float* ws, hipStream_t st) {
  return ssm_chunk_launch<T>(a, ws, st);
}

}  // namespace

extern "C" {

int64_t mqc_ssm_chunk_len_auto(int64_t batch, int64_t seq_len, int64_t d_inner,
                               int64_t d_state, int dtype) {
  if (batch < 0 || seq_len < 0 || d_inner < 0 || d_state < 0) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  return auto_chunk_len(batch, seq_len, d_inner, d_state);
}

int64_t mqc_ssm_chunked_workspace_bytes(int64_t batch, int64_t seq_len, int64_t d_inner,
                                        int64_t d_state, int64_t chunk_len) {
  if (batch < 0 || seq_len < 0 || d_inner < 0 || d_state < 0 || chunk_len < 1) return MQC_E_SHAPE;
  return ssm_chunk_workspace_bytes(batch, seq_len, d_inner, d_state, chunk_len);
}

int mqc_ssm_fused_fwd_chunked(const void* delta, const void* s, const void* B, const void* C,
                              const float* lambda_alpha, const float* lambda_imag, const float* D,
                              const void* h0, void* y, void* h_last, int64_t batch,
                              int64_t seq_len, int64_t d_inner, int64_t d_state,
                              int64_t chunk_len, float eps, int dtype, void* workspace,
                              int64_t workspace_bytes, void* stream) {
  bool nothing;
  int st = check_chunked(delta, s, B, C, lambda_alpha, lambda_imag, D, h0, y, h_last, batch,
                         seq_len, d_inner, d_state, chunk_len, dtype, nothing);
  if (st != MQC_OK || nothing) return st;
  SsmArgs a{};
  a.delta = delta; a.s = s; a.lam_alpha = lambda_alpha; a.lam_imag = lambda_imag; a.dvec = D;
  a.Bm = B; a.Cm = C; a.h0 = h0; a.y = y; a.h_last = h_last;
  a.batch = batch; a.T = seq_len; a.Dm = d_inner; a.S = d_state; a.eps = eps;
  const int64_t nc = seq_len > chunk_len ? (seq_len + chunk_len - 1) / chunk_len : 1;
  hipStream_t hs = (hipStream_t)stream;
  if (nc <= 1) {
    switch (dtype) {
      case MQC_F32: return launch_ssm<float, MODE_DL>(a, hs);
      case MQC_BF16: return launch_ssm<bf16_t, MODE_DL>(a, hs);
      default: return launch_ssm<f16_t, MODE_DL>(a, hs);
    }
  }
  if (d_state > kChunkMaxState) return MQC_E_LIMIT;
  if (batch * nc > 65535 || seq_len >= ((int64_t)1 << 30)) return MQC_E_LIMIT;
  const int64_t need = ssm_chunk_workspace_bytes(batch, seq_len, d_inner, d_state, chunk_len);
  if (!workspace) return MQC_E_NULL;
  if (workspace_bytes < need) return MQC_E_SPACE;
  if (!aligned(workspace, 16)) return MQC_E_ALIGN;
  a.chunk_len = chunk_len;
  a.n_chunks = nc;
  switch (dtype) {
    case MQC_F32: return run_chunked<float>(a, (float*)workspace, hs);
    case MQC_BF16: return run_chunked<bf16_t>(a, (float*)workspace, hs);
    default: return run_chunked<f16_t>(a, (float*)workspace, hs);
  }
}

int64_t mqc_ssm_chunked_scratch_bytes(void) { return kScratchBytes; }

int mqc_ssm_noalloc_prepare(void) {
  void* p = nullptr;
  return scratch_ptr(&p);
}

int mqc_ssm_fused_fwd_chunked_noalloc(const void* delta, const void* s, const void* B,
                                      const void* C, const float* lambda_alpha,
                                      const float* lambda_imag, const float* D, const void* h0,
                                      void* y, void* h_last, int64_t batch, int64_t seq_len,
                                      int64_t d_inner, int64_t d_state, int64_t chunk_len,
                                      float eps, int dtype, void* stream) {
  bool nothing;
  int st = check_chunked(delta, s, B, C, lambda_alpha, lambda_imag, D, h0, y, h_last, batch,
                         seq_len, d_inner, d_state, chunk_len, dtype, nothing);
  if (st != MQC_OK || nothing) return st;
  const int64_t nc = seq_len > chunk_len ? (seq_len + chunk_len - 1) / chunk_len : 1;
  if (nc > 1 && d_state > kChunkMaxState) return MQC_E_LIMIT;
  const int64_t need = ssm_chunk_workspace_bytes(batch, seq_len, d_inner, d_state, chunk_len);
  if (need > kScratchBytes) return MQC_E_SPACE;
  void* ws = nullptr;
  if (nc > 1) {
    st = scratch_ptr(&ws);
    if (st != MQC_OK) return st;
  }
  return mqc_ssm_fused_fwd_chunked(delta, s, B, C, lambda_alpha, lambda_imag, D, h0, y, h_last,
                                   batch, seq_len, d_inner, d_state, chunk_len, eps, dtype, ws,
                                   kScratchBytes, stream);
}

}  // extern "C"
