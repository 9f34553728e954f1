/*
 * mambaqc_hip.h — C ABI of libmambaqc_hip.so, the MI355X (gfx950) kernels of
 * the Quaternion Mamba-2 SSM hot path.
 *
 * Conventions shared by every entry point
 *   - All tensor arguments are device pointers to contiguous, row-major
 *     buffers owned by the caller. Nothing is allocated inside the library.
 *   - Outputs share no bytes with inputs, except where an entry point names an
 *     in-place form (such as h_last == h0 for a walk's state, out == x for the
 *     output step); the overlaps a launch could race on are checked where its
 *     comment says so and refused with MQC_E_OVERLAP.
 *   - A quaternion is four consecutive elements (w, x, y, z).
 *   - `dtype` selects the storage type of the tensors named in each comment:
 *     MQC_F32, MQC_BF16 or MQC_F16. Arithmetic is always fp32. Parameter
 *     arrays typed `const float*` are fp32 whatever `dtype` is.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream). Every call
 *     only enqueues work; it never synchronises.
 *   - The return value is MQC_OK (0), a negative MQC_E_* code when argument
 *     validation fails (checked before any HIP call, so these are safe to
 *     probe without a GPU), or a positive hipError_t from the launch.
 *   - No global mutable state: calls are re-entrant and thread-safe. The one
 *     exception is mqc_ssm_fused_fwd_chunked_noalloc (a fixed device array
 *     shared by its calls on one device).
 *
 * Each function names the reference interface (polux06/mambaqc) it replaces.
 */
#ifndef MAMBAQC_HIP_H
#define MAMBAQC_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MQC_F32 0
#define MQC_BF16 1
#define MQC_F16 2

#define MQC_OK 0
#define MQC_E_NULL (-1)      /* a required pointer is NULL */
#define MQC_E_SHAPE (-2)     /* a size is negative or inconsistent */
#define MQC_E_DTYPE (-3)     /* unknown dtype code */
#define MQC_E_ALIGN (-4)     /* a pointer is not aligned for the vector loads */
#define MQC_E_LIMIT (-5)     /* a size is beyond what the kernels support (for the
                              * SSM entry points: seq_len >= 2^30, d_state above the
                              * stated maximum, one (b, t) slice of B/C of 2 GiB or
                              * more, or a negative or too large D stride) */
#define MQC_E_SPACE (-6)     /* a workspace is smaller than the call needs */
#define MQC_E_OVERLAP (-7)   /* an output overlaps an input that the launch still reads
                              * (the chunked SSM walks: h_last over h0, dh0 over
                              * dh_last; every SSM walk: h_last sharing bytes with h0
                              * without being the same buffer; the fused output step:
                              * out over y, W, bias, z or a shifted x) */

/* Human-readable text for a status code (static storage, never NULL). */
const char* mqc_status_string(int status);

/* ABI version: bumped whenever a signature or an argument's meaning changes. */
int mqc_abi_version(void);

/* out = p (x) q, Hamilton product of n_quat quaternions. p, q, out: dtype.
 * Replaces quaternion_multiply, mambaqc/kernels/quaternion_ops.py:259-303
 * (and quaternion_multiply_batched, :306-357, which computes the same thing). */
int mqc_quaternion_multiply(const void* p, const void* q, void* out, int64_t n_quat,
                            int dtype, void* stream);

/* out = conj(q). Replaces quaternion_conjugate, quaternion_ops.py:360-391. */
int mqc_quaternion_conjugate(const void* q, void* out, int64_t n_quat, int dtype, void* stream);

/* out = conj(q) / max(|q|^2, eps). Replaces quaternion_inverse, quaternion_ops.py:394-428. */
int mqc_quaternion_inverse(const void* q, void* out, int64_t n_quat, float eps, int dtype,
                           void* stream);

/* out[i] = |q_i| (n_quat scalars). Replaces quaternion_norm, quaternion_ops.py:431-461. */
int mqc_quaternion_norm(const void* q, void* out, int64_t n_quat, int dtype, void* stream);

/* q = (1 - z/2)^-1 (x) (1 + z/2) per quaternion, the inverse taken as
 * conj/max(|.|^2, eps). z, q: dtype, n_quat quaternions.
 * Replaces cayley_discretization_fused, mambaqc/kernels/cayley_transform.py:132-195. */
int mqc_cayley_fwd(const void* z, void* q, int64_t n_quat, float eps, int dtype, void* stream);

/* Inclusive left-ordered cumulative Hamilton product along the seq axis:
 *   out[b,t,l] = q[b,t,l] (x) out[b,t-1,l],  out[b,-1,l] = 1.
 * q, out: dtype, shape [batch, seq_len, lanes, 4]; lanes = d_model * d_state
 * for the reference's [B,T,D,S,4] layout.
 * Replaces parallel_scan_quaternion, mambaqc/kernels/parallel_scan.py:171-264,
 * with the semantics of parallel_scan_quaternion_reference, :267-295. */
int mqc_cumprod_scan_fwd(const void* q, void* out, int64_t batch, int64_t seq_len,
                         int64_t lanes, int dtype, void* stream);

/* Quaternion SSM over a materialised evolution operator q:
 *   h_t = q_t (x) h_{t-1} + B_t (x) S_t      (S broadcast over d_state)
 *   y_t = sum_k C_{t,k} (x) h_{t,k} + D_t * S_t
 * q, B, C: dtype [batch, seq_len, d_inner, d_state, 4]; S: dtype
 * [batch, seq_len, d_inner, 4]; D: dtype, element (b,t,d) at
 * D[b*d_sb + t*d_st + d*d_sd] (strides in elements, 0 allowed, so an expanded
 * [d_inner] vector needs no copy); h0: dtype [batch, d_inner, d_state, 4] or
 * NULL for zeros; y: dtype [batch, seq_len, d_inner, 4]; h_last: dtype
 * [batch, d_inner, d_state, 4] or NULL. With seq_len 0, h_last (if given)
 * receives h0, or zeros, and the per-step operands may be NULL. h_last may be
 * h0; buffers that overlap without being the same are refused (MQC_E_OVERLAP).
 * Replaces ssm_forward_fused, mambaqc/kernels/ssm_fused.py:340-401, and (with
 * seq_len = 1, h0 = h_prev, h_last = h_new) ssm_step_fused, :258-337. */
int mqc_ssm_q_fwd(const void* q, const void* B, const void* S, const void* C, const void* D,
                  int64_t d_sb, int64_t d_st, int64_t d_sd, const void* h0, void* y,
                  void* h_last, int64_t batch, int64_t seq_len, int64_t d_inner,
                  int64_t d_state, int dtype, void* stream);

/* The block's fused SSM: Cayley discretisation of z = delta * Lambda computed
 * in registers, the recurrence above with S = (s, 0, 0, 0), and the k-reduction.
 *   Lambda[d,k] = (-softplus(lambda_alpha[d,k]), tanh(lambda_imag[d,k,0:3]))
 *   q_t = Cayley(delta[b,t,d] * Lambda[d,k]) with eps
 *   h_t = q_t (x) h_{t-1} + s[b,t,d] * B_t
 *   y_t = sum_k C_{t,k} (x) h_{t,k} + (D[d] * s[b,t,d], 0, 0, 0)
 * delta, s: dtype [batch, seq_len, d_inner]; B, C: dtype
 * [batch, seq_len, d_inner, d_state, 4]; lambda_alpha: fp32 [d_inner, d_state];
 * lambda_imag: fp32 [d_inner, d_state, 3]; D: fp32 [d_inner]; h0: fp32
 * [batch, d_inner, d_state, 4] or NULL; y: dtype [batch, seq_len, d_inner, 4];
 * h_last: fp32 [batch, d_inner, d_state, 4] or NULL. The state is carried in
 * fp32 whatever dtype is, so a walk split into pieces (recurrent decoding)
 * gives the same y as the whole walk. With seq_len 0, h_last (if given)
 * receives h0, or zeros; delta, s, B, C and y may then be NULL, the
 * parameters may not. h_last may be h0 (the state updated in place, as the
 * recurrent decode does): each state is written only by the lane that read it,
 * after its walk. Buffers that overlap without being the same are refused
 * (MQC_E_OVERLAP).
 * Replaces the body of QuaternionMamba2Block._ssm_forward,
 * mambaqc/models/quaternion_mamba2_block.py:206-228 (Lambda, z = delta*Lambda,
 * cayley_discretization_fused, ssm_forward_fused), without materialising z or q. */
int mqc_ssm_fused_fwd(const void* delta, const void* s, const void* B, const void* C,
                      const float* lambda_alpha, const float* lambda_imag, const float* D,
                      const void* h0, void* y, void* h_last, int64_t batch, int64_t seq_len,
                      int64_t d_inner, int64_t d_state, float eps, int dtype, void* stream);

/* Chunk length mqc_ssm_fused_fwd_chunked would be given by a caller that lets
 * the library choose: seq_len (one chunk, the whole walk) when batch * d_inner
 * * d_state states keep the GPU busy on their own, shorter chunks when they
 * do not: about 393216 / states chunks, each at least 64 steps, at most 1024
 * chunks and at most 65535 / batch (the chunked launches' limit on
 * batch * n_chunks). Negative: an MQC_E_* code. */
int64_t mqc_ssm_chunk_len_auto(int64_t batch, int64_t seq_len, int64_t d_inner,
                               int64_t d_state, int dtype);

/* Bytes of workspace mqc_ssm_fused_fwd_chunked needs for these sizes:
 * 24 * batch * (n_chunks - 1) * d_inner * d_state with n_chunks =
 * ceil(seq_len / chunk_len) (0 for one chunk). Negative: an MQC_E_* code. */
int64_t mqc_ssm_chunked_workspace_bytes(int64_t batch, int64_t seq_len, int64_t d_inner,
                                        int64_t d_state, int64_t chunk_len);

/* mqc_ssm_fused_fwd with the seq axis cut into chunks of chunk_len steps that
 * are walked side by side (the last chunk may be shorter): each chunk but the
 * last is first reduced to its transition (P = product of its q's, H = its end
 * state from zero), an associative scan over the chunks (the later transition
 * on the left) gives every chunk its start state, then every chunk is walked
 * from it. Same arguments and results as mqc_ssm_fused_fwd (h0, h_last fp32),
 * up to rounding; for batches too small to fill the GPU through
 * batch * d_inner * d_state alone. workspace: device memory of at least
 * mqc_ssm_chunked_workspace_bytes (16-byte aligned; may be NULL when
 * chunk_len >= seq_len), owned by the caller, no contents needed on entry.
 * d_state <= 64 when there is more than one chunk; batch * n_chunks <= 65535.
 * Unlike the whole walk, with more than one chunk h_last may not overlap h0
 * (MQC_E_OVERLAP): chunk 0 reads h0 while the last chunk writes h_last.
 * Replaces, like mqc_ssm_fused_fwd, mambaqc/models/quaternion_mamba2_block.py:206-228
 * (the sequential walk of kernels/ssm_fused.py:363-379); the chunked order of
 * evaluation follows the associative-scan idea of kernels/parallel_scan.py:171-264. */
int mqc_ssm_fused_fwd_chunked(const void* delta, const void* s, const void* B, const void* C,
                              const float* lambda_alpha, const float* lambda_imag, const float* D,
                              const void* h0, void* y, void* h_last, int64_t batch,
                              int64_t seq_len, int64_t d_inner, int64_t d_state,
                              int64_t chunk_len, float eps, int dtype, void* workspace,
                              int64_t workspace_bytes, void* stream);

/* mqc_ssm_fused_fwd_chunked without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * The chunk transitions go to a fixed device array inside the library,
 * mqc_ssm_chunked_scratch_bytes() bytes (32 MiB) on every device the library
 * runs on, held until the process ends; a call whose
 * mqc_ssm_chunked_workspace_bytes exceeds it returns MQC_E_SPACE before any
 * HIP call. Nothing is allocated or freed. Every call on one device uses the
 * same array, so calls that overlap on one device (concurrent streams,
 * threads) race: serialise them. No contents are needed on entry (every
 * transition is written before it is read). Otherwise as
 * mqc_ssm_fused_fwd_chunked. */
int mqc_ssm_fused_fwd_chunked_noalloc(const void* delta, const void* s, const void* B,
                                      const void* C, const float* lambda_alpha,
                                      const float* lambda_imag, const float* D, const void* h0,
                                      void* y, void* h_last, int64_t batch, int64_t seq_len,
                                      int64_t d_inner, int64_t d_state, int64_t chunk_len,
                                      float eps, int dtype, void* stream);

/* Size in bytes of the fixed device scratch of mqc_ssm_fused_fwd_chunked_noalloc. */
int64_t mqc_ssm_chunked_scratch_bytes(void);

/* Looks up the current device's address of that scratch, which
 * mqc_ssm_fused_fwd_chunked_noalloc otherwise looks up (hipGetSymbolAddress)
 * on its first call on each device. Call it once per device, with the device
 * current, before capturing no-alloc calls into a HIP graph, so that the
 * captured calls make no HIP runtime call but their kernel launches.
 * Idempotent and thread-safe. Returns MQC_OK or a hipError_t. No counterpart
 * in the reference. */
int mqc_ssm_noalloc_prepare(void);

/* The block's B and C projections fused with its SSM (mqc_ssm_fused_fwd) in one
 * launch, 16-bit storage (dtype MQC_BF16 or MQC_F16, for x, the weights, delta, s and
 * y; MQC_F32 is refused): B = x . B_weight^T and C = x . C_weight^T, viewed as
 * [batch, seq_len, d_inner, d_state, 4], are computed 256 tokens at a time by MFMA
 * tiles in LDS, rounded to dtype as the unfused projections store them, and
 * walked there, so neither is ever written to memory. x: [batch, seq_len, d_inner]
 * (the projections' input, 16-byte aligned); B_weight, C_weight: [d_inner * d_state * 4,
 * d_inner] (nn.Linear layout, 16-byte aligned); delta, s: [batch, seq_len, d_inner];
 * the parameters, h0, y and h_last as in mqc_ssm_fused_fwd (y 8-byte aligned, h0 and
 * h_last 16-byte aligned; h_last may be h0, a partial overlap is refused with
 * MQC_E_OVERLAP). d_inner a multiple of 64; d_state even,
 * at most 64. Replaces B_proj/C_proj (F.linear, mambaqc/layers/quaternion_linear.py:145-161,
 * called at mambaqc/models/quaternion_mamba2_block.py:186-191) together with the SSM
 * they feed (quaternion_mamba2_block.py:206-228). */
int mqc_ssm_fused_bc_fwd(const void* x, const void* B_weight, const void* C_weight,
                         const void* delta, const void* s, const float* lambda_alpha,
                         const float* lambda_imag, const float* D, const void* h0, void* y,
                         void* h_last, int64_t batch, int64_t seq_len, int64_t d_inner,
                         int64_t d_state, float eps, int dtype, void* stream);

/* Bytes of workspace mqc_ssm_fused_bc_fwd_split needs for these sizes: the two
 * halves' fp32 partial sums of y, 2 * batch * seq_len * d_inner * 16; 0 when there is
 * one half of states (d_state <= 32) or nothing to walk. Negative: an MQC_E_* code. */
int64_t mqc_ssm_fused_bc_split_workspace_bytes(int64_t batch, int64_t seq_len,
                                               int64_t d_inner, int64_t d_state);

/* mqc_ssm_fused_bc_fwd with each half of the states (32) in a workgroup of its own,
 * for batches too small to share the weight rows: a workgroup per (b, d) streams its
 * d's 512 weight rows once per 256-token tile, the workgroups of a d's batches share
 * those reads in L2, and a single sequence's resident d's want more weight rows than the
 * Infinity Cache holds; per half they want half as many. Each half writes its fp32
 * partial sum of y to the workspace (at least
 * mqc_ssm_fused_bc_split_workspace_bytes, 16-byte aligned, owned by the caller, no
 * contents needed on entry) and a second launch adds them with D s, in the order the
 * one-launch form does: y equals mqc_ssm_fused_bc_fwd's bit for bit. With one half of
 * states the call is mqc_ssm_fused_bc_fwd (workspace unused, may be NULL). Same
 * arguments, limits and replaced reference lines as mqc_ssm_fused_bc_fwd. */
int mqc_ssm_fused_bc_fwd_split(const void* x, const void* B_weight, const void* C_weight,
                               const void* delta, const void* s, const float* lambda_alpha,
                               const float* lambda_imag, const float* D, const void* h0,
                               void* y, void* h_last, int64_t batch, int64_t seq_len,
                               int64_t d_inner, int64_t d_state, float eps, int dtype,
                               void* workspace, int64_t workspace_bytes, void* stream);

/* The block's output step in one launch, bf16 only (dtype MQC_BF16):
 *   out[r, n] = x[r, n] + sigmoid(z[r, n]) * bf16(sum_j y[r, j] W[n, j] + bias[n])
 * for r < rows, n < d_model: the quaternion -> real projection out_proj of the
 * QuaternionLayerNorm output y [rows, k] (k = 4 * d_inner, components innermost) by
 * W [d_model, k] (+ bias [d_model] or NULL), rounded to bf16 as the projection stores
 * it, gated by z [rows, >= d_model] (row stride z_row_stride elements, read in place:
 * the gate half of in_proj's output) and added to the residual x [rows, d_model].
 * y, W, x, z, out 16-byte aligned; d_model a multiple of 8, k of 64, z_row_stride of 8.
 * out may be x itself (an in-place residual); out sharing bytes with y, W, bias, z or
 * with x without being x is refused (MQC_E_OVERLAP): other tiles still read them.
 * Replaces out_proj (QuaternionLinear._forward_quaternion_to_real,
 * mambaqc/layers/quaternion_linear.py:163-172) with the gate and residual of
 * mambaqc/models/quaternion_mamba2_block.py:157-164 (z[..., :d_model], as the
 * reference's Lite block gates), which mqc_out_gate_fwd covers unfused. */
int mqc_out_proj_gate_fwd(const void* y, const void* W, const void* bias, const void* x,
                          const void* z, int64_t z_row_stride, void* out, int64_t rows,
                          int64_t d_model, int64_t k, int dtype, void* stream);

/* C[M, N] = X[M, K] . W[N, K]^T in bf16 or fp16 (dtype MQC_BF16 or MQC_F16) with
 * fp32 accumulation, contiguous row-major X, W, C, 16-byte aligned; N a multiple of
 * 256, K of 64, M any. The hand-written MFMA GEMM of the block's B/C
 * projections (F.linear, mambaqc/layers/quaternion_linear.py:145-161, called
 * at mambaqc/models/quaternion_mamba2_block.py:186-191), the first stage of
 * fusing them with the SSM walk; the block itself keeps hipBLASLt, which is
 * faster at the config-3 shape. */
int mqc_gemm_nt(const void* X, const void* W, void* C, int64_t M, int64_t N, int64_t K, int dtype,
                void* stream);

/* Y[M, N] = X[M, K] . W[N, K]^T (+ bias[N]) for few rows (M <= 16, a decode
 * step's tokens), dtype MQC_BF16 or MQC_F16, fp32 accumulation: the F.linear of
 * an nn.Linear / QuaternionLinear (mambaqc/layers/quaternion_linear.py:145-172;
 * the block's layers, mambaqc/models/quaternion_mamba2_block.py:78-122) in the
 * recurrent decode. A second weight sharing X (W2, bias2, Y2, N2 > 0) runs in
 * the same launch; N2 = 0 for one. X dense [M, K], 16-byte aligned; W1, W2
 * dense [N, K], 16-byte aligned; bias1, bias2 dtype [N] or NULL; Y1, Y2 dense
 * [M, N]. K must be a positive multiple of 32 with M * (K + 8) * 2 <= 65536
 * (MQC_E_LIMIT otherwise: the caller uses another GEMM). */
int mqc_gemm_skinny_nt(const void* X, int64_t M, int64_t K, const void* W1, const void* bias1,
                       void* Y1, int64_t N1, const void* W2, const void* bias2, void* Y2,
                       int64_t N2, int dtype, void* stream);

/* Quaternion LayerNorm over the d axis of each of `rows` rows of d quaternions:
 *   n = sqrt(|q|^2 + eps); mu, var = mean and biased variance of n over d;
 *   out = gamma * (n - mu) / sqrt(var + eps) * q / (n + eps) + beta.
 * q, out: dtype [rows, d, 4]; gamma: fp32 [d]; beta: fp32 [d, 4];
 * mean, rstd: fp32 [rows] or NULL (saved statistics).
 * Replaces quaternion_layer_norm_fused / QuaternionLayerNorm.forward,
 * mambaqc/kernels/quaternion_norm.py:119-215, with the semantics of
 * quaternion_layer_norm_reference, :219-245. */
int mqc_qln_fwd(const void* q, const float* gamma, const float* beta, void* out, float* mean,
                float* rstd, int64_t rows, int64_t d, float eps, int dtype, void* stream);

/* Front of the block: depthwise causal conv1d (kernel `kernel` <= 8, left zero
 * padding) fused with SiLU:
 *   out[b,t,c] = silu(bias[c] + sum_j w[c,j] * x[b, t-(kernel-1)+j, c])
 * x: dtype, element (b,t,c) at x[(b*seq_len + t) * x_row_stride + c] (the first
 * half of in_proj's output is read in place); w: fp32 [channels, kernel]; bias:
 * fp32 [channels] or NULL; out: dtype dense [batch, seq_len, channels]. (16-byte
 * accesses when channels and x_row_stride are multiples of 16 / sizeof(dtype)
 * and the pointers are 16-byte aligned; element accesses otherwise.)
 * Replaces CausalConv1d.forward + F.silu, mambaqc/layers/causal_conv1d.py:68-91
 * and mambaqc/models/quaternion_mamba2_block.py:141-144. */
int mqc_causal_conv_silu_fwd(const void* x, int64_t x_row_stride, const float* w, const float* bias,
                             void* out, int64_t batch, int64_t seq_len, int64_t channels,
                             int64_t kernel, int dtype, void* stream);

/* Steps per thread (R) of the conv kernels: the backward's weight partials have
 * batch * ceil(seq_len / R) rows. */
int mqc_conv_run_length(void);

/* Backward of mqc_causal_conv_silu_fwd given gout (dtype dense [batch, seq_len,
 * channels]): dx (dtype, rows dx_row_stride apart); dw_part fp32
 * [batch * ceil(seq_len / R), channels, kernel] and dbias_part fp32
 * [batch * ceil(seq_len / R), channels], R = mqc_conv_run_length(), to be
 * summed over the first axis by the caller. */
int mqc_causal_conv_silu_bwd(const void* x, int64_t x_row_stride, const float* w,
                             const float* bias, const void* gout, void* dx, int64_t dx_row_stride,
                             float* dw_part, float* dbias_part, int64_t batch, int64_t seq_len,
                             int64_t channels, int64_t kernel, int dtype, void* stream);

/* One step of mqc_causal_conv_silu_fwd for recurrent decoding: one new row per
 * batch row, x: dtype, element (b,c) at x[b * x_row_stride + c]; tail: dtype
 * dense [batch, kernel-1, channels], the kernel-1 inputs before x, oldest first
 * (may be NULL when kernel == 1). Writes out (dtype dense [batch, channels]) =
 * silu(bias[c] + sum_{j<kernel-1} w[c,j] * tail[b,j,c] + w[c,kernel-1] * x[b,c]),
 * the forward's value for that row with the same order of operations, and then
 * updates tail in place to the last kernel-1 inputs including x (bit copies).
 * The reference has no recurrent decode: its generate() reruns CausalConv1d.forward
 * over the whole sequence for every new token (mambaqc/models/quaternion_mamba2.py:192-225,
 * mambaqc/layers/causal_conv1d.py:68-91); this replaces the concatenation of the
 * cached tail with the new row and that conv in the one-token step. */
int mqc_causal_conv_silu_step(const void* x, int64_t x_row_stride, void* tail, const float* w,
                              const float* bias, void* out, int64_t batch, int64_t channels,
                              int64_t kernel, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Training: forward with state checkpoints, and the backward passes.
 * The reference has no backward for any of its GPU kernels (its Triton launches
 * sit outside autograd); these entry points serve torch.autograd.Function
 * wrappers whose gradients equal autograd through the reference's CPU path
 * (models/quaternion_mamba2_block.py:124-230 with kernels/ssm_fused.py:405-430,
 * kernels/quaternion_norm.py:219-245).
 * ------------------------------------------------------------------------- */

/* Checkpoint interval K that mqc_ssm_fused_bwd requires for `dtype` (the
 * backward keeps K steps of operands and states in registers). */
int mqc_ssm_bwd_ckpt_every(int dtype);

/* mqc_ssm_fused_fwd (h0, h_last fp32) plus fp32 state checkpoints for the backward:
 * h_ckpt [batch, ceil(seq_len / ckpt_every), d_inner, d_state, 4] receives the
 * state at the last step of every chunk of ckpt_every steps (the last chunk may
 * be shorter). With seq_len 0 it has no entries and may be NULL. */
int mqc_ssm_fused_fwd_train(const void* delta, const void* s, const void* B, const void* C,
                            const float* lambda_alpha, const float* lambda_imag, const float* D,
                            const void* h0, void* y, void* h_last, float* h_ckpt,
                            int64_t ckpt_every, int64_t batch, int64_t seq_len, int64_t d_inner,
                            int64_t d_state, float eps, int dtype, void* stream);

/* Backward of mqc_ssm_fused_fwd_train given gy = dL/dy (dtype [batch, seq_len,
 * d_inner, 4]) and optionally dh_last = dL/dh_last (fp32 [batch, d_inner,
 * d_state, 4]). Writes d_delta, d_s (fp32 [batch, seq_len, d_inner]: these
 * sums over d_state keep fp32 precision for callers whose delta is fp32, as
 * under autocast), dB, dC (dtype, shape of B), per-batch partial parameter gradients
 * dlambda_alpha_part fp32 [batch, d_inner, d_state],
 * dlambda_imag_part fp32 [batch, d_inner, d_state, 3], dD_part fp32
 * [batch, d_inner] (the caller sums them over batch), and dh0 (fp32
 * [batch, d_inner, d_state, 4]) if non-NULL. h0 (fp32) and h_ckpt must be the forward's;
 * ckpt_every must equal mqc_ssm_bwd_ckpt_every(dtype); d_state <= 64. With
 * seq_len 0 the partials are zeros and dh0 = dh_last (zeros without it); the
 * per-step tensors and h_ckpt may then be NULL. */
int mqc_ssm_fused_bwd(const void* delta, const void* s, const void* B, const void* C,
                      const float* lambda_alpha, const float* lambda_imag, const float* D,
                      const void* h0, const float* h_ckpt, int64_t ckpt_every, const void* gy,
                      const void* dh_last, float* d_delta, float* d_s, void* dB, void* dC,
                      float* dlambda_alpha_part, float* dlambda_imag_part, float* dD_part,
                      void* dh0, int64_t batch, int64_t seq_len, int64_t d_inner,
                      int64_t d_state, float eps, int dtype, void* stream);

/* mqc_ssm_fused_fwd_train with the seq axis cut into chunks of chunk_len steps
 * walked side by side (for batch x d_inner x d_state too small to fill the GPU,
 * as in mqc_ssm_fused_fwd_chunked). chunk_len must be a multiple of ckpt_every
 * (the checkpoints are the whole walk's, at the same steps); workspace holds
 * mqc_ssm_chunked_workspace_bytes(batch, seq_len, d_inner, d_state, chunk_len)
 * bytes (16-byte aligned; MQC_E_SPACE if smaller); d_state <= 64. chunk_len >=
 * seq_len is the whole walk (no workspace used). With more than one chunk
 * h_last may not overlap h0 (MQC_E_OVERLAP). No counterpart in the
 * reference (its GPU path has no training forward). */
int mqc_ssm_fused_fwd_train_chunked(const void* delta, const void* s, const void* B,
                                    const void* C, const float* lambda_alpha,
                                    const float* lambda_imag, const float* D, const void* h0,
                                    void* y, void* h_last, float* h_ckpt, int64_t ckpt_every,
                                    int64_t batch, int64_t seq_len, int64_t d_inner,
                                    int64_t d_state, int64_t chunk_len, float eps, int dtype,
                                    void* workspace, int64_t workspace_bytes, void* stream);

/* mqc_ssm_fused_bwd with the seq axis cut into chunks of chunk_len steps run
 * side by side: the adjoint entering each chunk comes from a reverse carry
 * pass over the chunks after it (same workspace size and chunk_len rule as
 * mqc_ssm_fused_fwd_train_chunked). With n_chunks = ceil(seq_len / chunk_len)
 * > 1 the parameter partials have n_chunks * batch rows
 * (dlambda_alpha_part fp32 [n_chunks * batch, d_inner, d_state], and so on; the
 * caller sums the first axis); chunk_len >= seq_len is mqc_ssm_fused_bwd.
 * With more than one chunk dh0 may not overlap dh_last (MQC_E_OVERLAP). No
 * counterpart in the reference. */
int mqc_ssm_fused_bwd_chunked(const void* delta, const void* s, const void* B, const void* C,
                              const float* lambda_alpha, const float* lambda_imag, const float* D,
                              const void* h0, const float* h_ckpt, int64_t ckpt_every,
                              const void* gy, const void* dh_last, float* d_delta, float* d_s,
                              void* dB, void* dC, float* dlambda_alpha_part,
                              float* dlambda_imag_part, float* dD_part, void* dh0, int64_t batch,
                              int64_t seq_len, int64_t d_inner, int64_t d_state,
                              int64_t chunk_len, float eps, int dtype, void* workspace,
                              int64_t workspace_bytes, void* stream);

/* Backward of mqc_qln_fwd given dout (dtype [rows, d, 4]) and the forward's
 * saved mean and rstd: writes dq (dtype [rows, d, 4]) and
 * ne = n-hat * <dout, q / (n + eps)> (fp32 [rows, d]); dgamma = sum over rows
 * of ne and dbeta = sum over rows of dout are left to the caller. */
int mqc_qln_bwd(const void* q, const void* dout, const float* gamma, const float* mean,
                const float* rstd, void* dq, float* ne, int64_t rows, int64_t d, float eps,
                int dtype, void* stream);

/* Backward of mqc_out_gate_fwd (dx = dout is the caller's). z is read as in the
 * forward (first `cols` columns, rows z_row_stride apart); dz (dtype, dense
 * [rows, z_cols], z_cols >= cols) = dout * y_real * sigmoid'(z) in the first
 * `cols` columns and 0 after them; dy_real (dtype [rows, cols]) =
 * dout * sigmoid(z). */
int mqc_out_gate_bwd(const void* dout, const void* z, int64_t z_row_stride, const void* y_real,
                     void* dz, void* dy_real, int64_t rows, int64_t cols, int64_t z_cols,
                     int dtype, void* stream);

/* Output step epilogue of the block: out = x + sigmoid(z) * y_real, where
 * x, y_real, out: dtype [rows, cols] contiguous and z: dtype with element
 * (r, c) at z[r * z_row_stride + c] (the gate half of in_proj's output).
 * Replaces mambaqc/models/quaternion_mamba2_block.py:159-164 (gating + residual),
 * with the gate sliced to the first d_model features as in
 * mambaqc/models/quaternion_mamba2_lite_block.py:163. */
int mqc_out_gate_fwd(const void* x, const void* z, int64_t z_row_stride, const void* y_real,
                     void* out, int64_t rows, int64_t cols, int dtype, void* stream);

/* Front of the block's SSM over n elements of same-shaped contiguous tensors:
 *   delta = softplus(dt_raw)   (identity above 20, torch's threshold)
 *   s     = sigmoid(g_raw) * x
 * dt_raw, g_raw, x, delta, s: dtype. dt_raw is dt_proj's output (bias added),
 * g_raw gate_proj's. Replaces mambaqc/models/quaternion_mamba2_block.py:183
 * (Delta = F.softplus(self.dt_proj(x))) and :197-198 (gate * x). */
int mqc_ssm_front_fwd(const void* dt_raw, const void* g_raw, const void* x, void* delta, void* s,
                      int64_t n, int dtype, void* stream);

/* Backward of mqc_ssm_front_fwd from fp32 d_delta, d_s [n]:
 *   d_dt_raw = d_delta * sigmoid(dt_raw) (d_delta above 20),
 *   d_g_raw = d_s * x * sigmoid'(g_raw),  d_x = d_s * sigmoid(g_raw)
 * (d_x is the part of x's gradient that flows through s). Outputs: dtype [n].
 * The reference runs these through torch autograd (same lines as the forward). */
int mqc_ssm_front_bwd(const void* dt_raw, const void* g_raw, const void* x, const float* d_delta,
                      const float* d_s, void* d_dt_raw, void* d_g_raw, void* d_x, int64_t n,
                      int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MAMBAQC_HIP_H */
