// Front of the block: depthwise causal conv1d (kernel K, left zero padding)
// fused with SiLU, forward and backward
// (mambaqc/layers/causal_conv1d.py:68-91 followed by F.silu,
//  mambaqc/models/quaternion_mamba2_block.py:141-144).
//
//   pre[b,t,c] = bias[c] + sum_{j<K} w[c,j] * x[b, t-(K-1)+j, c]   (x = 0 for t < 0)
//   out[b,t,c] = silu(pre) = pre * sigmoid(pre)
//
// x is read in place with a row stride (the first half of in_proj's output,
// [B, T, 2*C]); out is a dense [B, T, C]. One thread owns V consecutive
// channels (16 bytes of storage, or one element when the layout does not
// allow vectors) of one batch row for a run of TR consecutive steps and slides
// a K-row window along t, so every input row is loaded once per run (plus K-1
// rows of overlap) and every output row written once.
//
// Backward, given gout = dL/dout:
//   gp[b,t,c]  = gout * silu'(pre),  silu'(p) = sig(p) (1 + p (1 - sig(p)))
//   dx[b,t,c]  = sum_j w[c,j] * gp[b, t+(K-1)-j, c]          (gp = 0 past T)
//   dw[c,j]    = sum_{b,t} gp[b,t,c] * x[b, t-(K-1)+j, c]
//   dbias[c]   = sum_{b,t} gp[b,t,c]
// pre is recomputed from x. dw and dbias are written as partial sums per
// (b, run) that the caller adds up.
#include "common.hpp"

namespace mqc {

constexpr int kConvThreads = 256;
constexpr int kConvMaxK = 8;

template <typename T>
constexpr int conv_vec() { return 16 / (int)sizeof(T); }

// Hardware exp and reciprocal (about 1 ulp each); the IEEE division would
// cost ten instructions per element in what is otherwise a few FMAs.
__device__ inline float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

// V consecutive elements: one 16-byte access, or V == 1 (any alignment).
template <typename T, int V>
__device__ inline void ld(const T* __restrict__ p, float (&r)[V]) {
  if constexpr (V == 1) r[0] = load_scalar(p);
  else load_vec<T, V>(p, r);
}
template <typename T, int V>
__device__ inline void st(T* __restrict__ p, const float (&r)[V]) {
  if constexpr (V == 1) store_scalar(p, r[0]);
  else store_vec<T, V>(p, r);
}

// Load V channels of row t (zeros outside [0, T)). The row is clamped onto a
// valid one and the value masked, so the load carries no predicate and the
// loads of a run issue back to back.
template <typename T, int V>
__device__ inline void conv_row(const T* __restrict__ x, int64_t xs, int64_t b, int64_t T_len,
                                int64_t t, int64_t c, float (&r)[V]) {
  const bool in = t >= 0 && t < T_len;
  const int64_t tc = t < 0 ? 0 : (t < T_len ? t : T_len - 1);
  ld<T, V>(x + (b * T_len + tc) * xs + c, r);
#pragma unroll
  for (int v = 0; v < V; ++v) r[v] = in ? r[v] : 0.f;
}

template <typename T, int K, int TR, int V>
__global__ __launch_bounds__(kConvThreads) void conv_silu_fwd_kernel(
    const T* __restrict__ x, int64_t xs, const float* __restrict__ w, const float* __restrict__ bias,
    T* __restrict__ out, int64_t Bn, int64_t T_len, int64_t C) {
  const int64_t cv = C / V;                       // channel vectors per row
  const int64_t runs = (T_len + TR - 1) / TR;
  const int64_t item = (int64_t)blockIdx.x * kConvThreads + threadIdx.x;
  if (item >= Bn * runs * cv) return;
  const int64_t c = (item % cv) * V;
  const int64_t br = item / cv;
  const int64_t b = br / runs;
  const int64_t t0 = (br - b * runs) * TR;

  float wk[K][V], bs[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    bs[v] = bias ? bias[c + v] : 0.f;
#pragma unroll
    for (int j = 0; j < K; ++j) wk[j][v] = w[(c + v) * K + j];
  }
  float win[K][V];  // win[j] = x[t - (K-1) + j]
#pragma unroll
  for (int j = 0; j < K - 1; ++j) conv_row<T, V>(x, xs, b, T_len, t0 - (K - 1) + j, c, win[j]);
#pragma unroll
  for (int i = 0; i < TR; ++i) {
    const int64_t t = t0 + i;
    conv_row<T, V>(x, xs, b, T_len, t, c, win[K - 1]);
    float o[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float p = bs[v];
#pragma unroll
      for (int j = 0; j < K; ++j) p = fmaf(wk[j][v], win[j][v], p);
      o[v] = p * sigmoid_f(p);
    }
    if (t < T_len) st<T, V>(out + (b * T_len + t) * C + c, o);
#pragma unroll
    for (int j = 0; j < K - 1; ++j)
#pragma unroll
      for (int v = 0; v < V; ++v) win[j][v] = win[j + 1][v];
  }
}

// One decode step: the conv over one new row per batch row, continued from the
// K-1 rows before it, which live in `tail` [B, K-1, C] (oldest first). Every
// thread owns one (b, c): out[b, c] is the forward's pre-activation over the
// window (tail rows, then x) in the same order, so a sequence fed step by step
// equals it fed whole; then the thread shifts its column of the tail by one
// row and appends x, as raw storage copies. Each thread reads its tail column
// before writing it and no two threads share one, so the update is in place.
//
// PACK: the rounding of the forward's 16-byte path, which the forward takes for
// whole sequences when C is a multiple of its vector width: the product
// p * sigmoid(p) rounded to fp32, then converted with the packed conversion.
// Without it the compiler fuses the product and the conversion to a 16-bit
// type into one instruction (one rounding), as the forward's element path
// does; the two can differ in the last bit of a 16-bit output.
template <typename T, int K, bool PACK>
__global__ __launch_bounds__(kConvThreads) void conv_silu_step_kernel(
    const T* __restrict__ x, int64_t xs, T* tail, const float* __restrict__ w,
    const float* __restrict__ bias, T* __restrict__ out, int64_t Bn, int64_t C) {
  const int64_t item = (int64_t)blockIdx.x * kConvThreads + threadIdx.x;
  if (item >= Bn * C) return;
  const int64_t b = item / C;
  const int64_t c = item - b * C;
  T* tc = tail + b * (K - 1) * C + c;
  const T xv = x[b * xs + c];
  T raw[K];
#pragma unroll
  for (int j = 0; j < K - 1; ++j) raw[j] = tc[j * C];
  raw[K - 1] = xv;
  float p = bias ? bias[c] : 0.f;
#pragma unroll
  for (int j = 0; j < K; ++j) p = fmaf(w[c * K + j], io<T>::to_f32(raw[j]), p);
  float o = p * sigmoid_f(p);
  if constexpr (PACK && sizeof(T) == 2) {
    asm volatile("" : "+v"(o));  // keep the product an fp32 value
    out[b * C + c].bits = (uint16_t)(pack2<T>(o, o) & 0xffffu);
  } else {
    store_scalar(out + b * C + c, o);
  }
#pragma unroll
  for (int j = 0; j < K - 1; ++j) tc[j * C] = raw[j + 1];
}

// Backward. Thread layout as the forward. dw_part / db_part: [Bn * runs, C, K]
// and [Bn * runs, C] (fp32).
template <typename T, int K, int TR, int V>
__global__ __launch_bounds__(kConvThreads) void conv_silu_bwd_kernel(
    const T* __restrict__ x, int64_t xs, const float* __restrict__ w, const float* __restrict__ bias,
    const T* __restrict__ gout, T* __restrict__ dx, int64_t dxs, float* __restrict__ dw_part,
    float* __restrict__ db_part, int64_t Bn, int64_t T_len, int64_t C) {
  const int64_t cv = C / V;
  const int64_t runs = (T_len + TR - 1) / TR;
  const int64_t item = (int64_t)blockIdx.x * kConvThreads + threadIdx.x;
  if (item >= Bn * runs * cv) return;
  const int64_t c = (item % cv) * V;
  const int64_t br = item / cv;
  const int64_t b = br / runs;
  const int64_t t0 = (br - b * runs) * TR;

  float wk[K][V], bs[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    bs[v] = bias ? bias[c + v] : 0.f;
#pragma unroll
    for (int j = 0; j < K; ++j) wk[j][v] = w[(c + v) * K + j];
  }
  float dwa[K][V], dba[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    dba[v] = 0.f;
#pragma unroll
    for (int j = 0; j < K; ++j) dwa[j][v] = 0.f;
  }
  // gp of the K-1 steps after the current one are needed for dx; walk t
  // downwards from the run's end so that they are at hand.
  const int64_t t_end = (t0 + TR < T_len ? t0 + TR : T_len);
  float gpw[K][V];  // gpw[j] = gp[t + j] (zero past T)
  // x window for the steps t-(K-1) .. t, filled per step (K loads, L2 hits).
  // Prime gp for t_end .. t_end + K - 2 (the next run's first steps).
#pragma unroll
  for (int j = 1; j < K; ++j) {
    const int64_t tt = t_end - 1 + j;
    const bool in = tt < T_len;
    const int64_t tc = in ? tt : T_len - 1;
    float xw[K][V];
#pragma unroll
    for (int q = 0; q < K; ++q) conv_row<T, V>(x, xs, b, T_len, tc - (K - 1) + q, c, xw[q]);
    float g[V];
    ld<T, V>(gout + (b * T_len + tc) * C + c, g);
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float p = bs[v];
#pragma unroll
      for (int q = 0; q < K; ++q) p = fmaf(wk[q][v], xw[q][v], p);
      const float sg = sigmoid_f(p);
      gpw[j][v] = in ? g[v] * sg * (1.f + p * (1.f - sg)) : 0.f;
    }
  }
#pragma unroll
  for (int i = TR - 1; i >= 0; --i) {
    const int64_t t = t0 + i;
    // Steps past T (the last run only) are computed on a clamped row and
    // discarded: they contribute nothing and do not shift the window.
    const bool live = t < T_len;
    const int64_t tc = live ? t : T_len - 1;
    float xw[K][V];
#pragma unroll
    for (int q = 0; q < K; ++q) conv_row<T, V>(x, xs, b, T_len, tc - (K - 1) + q, c, xw[q]);
    float g[V];
    ld<T, V>(gout + (b * T_len + tc) * C + c, g);
    if (!live) continue;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float p = bs[v];
#pragma unroll
      for (int q = 0; q < K; ++q) p = fmaf(wk[q][v], xw[q][v], p);
      const float sg = sigmoid_f(p);
      const float gp = g[v] * sg * (1.f + p * (1.f - sg));
      gpw[0][v] = gp;
      dba[v] += gp;
#pragma unroll
      for (int q = 0; q < K; ++q) dwa[q][v] = fmaf(gp, xw[q][v], dwa[q][v]);
    }
    float o[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      float s = 0.f;
      // x[t] feeds pre[t + (K-1) - j] through w[j]: dx[t] = sum_j w[j] gp[t + K-1-j].
#pragma unroll
      for (int j = 0; j < K; ++j) s = fmaf(wk[j][v], gpw[K - 1 - j][v], s);
      o[v] = s;
    }
    st<T, V>(dx + (b * T_len + t) * dxs + c, o);
#pragma unroll
    for (int j = K - 1; j > 0; --j)
#pragma unroll
      for (int v = 0; v < V; ++v) gpw[j][v] = gpw[j - 1][v];
  }
  float* dwp = dw_part + (br * C + c) * K;
#pragma unroll
  for (int v = 0; v < V; ++v) {
    db_part[br * C + c + v] = dba[v];
#pragma unroll
    for (int j = 0; j < K; ++j) dwp[v * K + j] = dwa[j][v];
  }
}

constexpr int kConvRun = 16;  // steps per thread (the backward's partial sums come per run)
constexpr int kConvRunShort = 4;
// Forward threads below which the short run is used: 4 waves per SIMD of the
// 256 CUs. Short runs re-read K-1 rows per run (from L2) but give the small
// launches (decoding, short prompts, config 3's 98 304 long runs) more waves
// to hide latency with.
constexpr int64_t kConvShortBelow = 256LL * 4 * 4 * 64;

template <typename T, int K, int V>
int launch_conv_kv(bool bwd, const void* x, int64_t xs, const float* w, const float* bias,
                   const void* gout, void* out_or_dx, int64_t dxs, float* dw_part, float* db_part,
                   int64_t Bn, int64_t T_len, int64_t C, hipStream_t s) {
  const int64_t runs = (T_len + kConvRun - 1) / kConvRun;
  const int64_t items = Bn * runs * (C / V);
  const int64_t blocks = (items + kConvThreads - 1) / kConvThreads;
  if (blocks > 0x7fffffffLL) return MQC_E_LIMIT;
  if (!bwd && items < kConvShortBelow) {
    const int64_t items_s = Bn * ((T_len + kConvRunShort - 1) / kConvRunShort) * (C / V);
    const int64_t blocks_s = (items_s + kConvThreads - 1) / kConvThreads;
    conv_silu_fwd_kernel<T, K, kConvRunShort, V><<<dim3((unsigned)blocks_s), dim3(kConvThreads),
                                                   0, s>>>((const T*)x, xs, w, bias,
                                                           (T*)out_or_dx, Bn, T_len, C);
  } else if (!bwd)
    conv_silu_fwd_kernel<T, K, kConvRun, V><<<dim3((unsigned)blocks), dim3(kConvThreads), 0, s>>>(
        (const T*)x, xs, w, bias, (T*)out_or_dx, Bn, T_len, C);
  else
    conv_silu_bwd_kernel<T, K, kConvRun, V><<<dim3((unsigned)blocks), dim3(kConvThreads), 0, s>>>(
        (const T*)x, xs, w, bias, (const T*)gout, (T*)out_or_dx, dxs, dw_part, db_part, Bn, T_len,
        C);
  return launch_status();
}

// 16-byte accesses when the channel count, the row strides and the pointers
// allow them; one element per thread otherwise.
template <typename T, int K>
int launch_conv_k(bool bwd, const void* x, int64_t xs, const float* w, const float* bias,
                  const void* gout, void* out_or_dx, int64_t dxs, float* dw_part, float* db_part,
                  int64_t Bn, int64_t T_len, int64_t C, hipStream_t s) {
  constexpr int V = conv_vec<T>();
  const bool wide = C % V == 0 && xs % V == 0 && (!bwd || dxs % V == 0) && aligned(x, 16) &&
                    aligned(out_or_dx, 16) && (!bwd || aligned(gout, 16));
  if (wide)
    return launch_conv_kv<T, K, V>(bwd, x, xs, w, bias, gout, out_or_dx, dxs, dw_part, db_part,
                                   Bn, T_len, C, s);
  return launch_conv_kv<T, K, 1>(bwd, x, xs, w, bias, gout, out_or_dx, dxs, dw_part, db_part, Bn,
                                 T_len, C, s);
}

template <typename T>
int launch_conv(bool bwd, const void* x, int64_t xs, const float* w, const float* bias,
                const void* gout, void* out_or_dx, int64_t dxs, float* dw_part, float* db_part,
                int64_t Bn, int64_t T_len, int64_t C, int64_t K, hipStream_t s) {
  if (Bn == 0 || T_len == 0 || C == 0) return MQC_OK;
  if (!aligned(x, sizeof(T)) || !aligned(out_or_dx, sizeof(T)) || (bwd && !aligned(gout, sizeof(T))) ||
      !aligned(w, 4) || (bias && !aligned(bias, 4)))
    return MQC_E_ALIGN;
  switch (K) {
    case 1: return launch_conv_k<T, 1>(bwd, x, xs, w, bias, gout, out_or_dx, dxs, dw_part, db_part, Bn, T_len, C, s);
    case 2: return launch_conv_k<T, 2>(bwd, x, xs, w, bias, gout, out_or_dx, dxs, dw_part, db_part, Bn, T_len, C, s);
    case 3: return launch_conv_k<T, 3>(bwd, x, xs, w, bias, gout, out_or_dx, dxs, dw_part, db_part, Bn, T_len, C, s);
    case 4: return launch_conv_k<T, 4>(bwd, x, xs, w, bias, gout, out_or_dx, dxs, dw_part, db_part, Bn, T_len, C, s);
    case 5: return launch_conv_k<T, 5>(bwd, x, xs, w, bias, gout, out_or_dx, dxs, dw_part, db_part, Bn, T_len, C, s);
    case 6: return launch_conv_k<T, 6>(bwd, x, xs, w, bias, gout, out_or_dx, dxs, dw_part, db_part, Bn, T_len, C, s);
    case 7: return launch_conv_k<T, 7>(bwd, x, xs, w, bias, gout, out_or_dx, dxs, dw_part, db_part, Bn, T_len, C, s);
    case 8: return launch_conv_k<T, 8>(bwd, x, xs, w, bias, gout, out_or_dx, dxs, dw_part, db_part, Bn, T_len, C, s);
    default: return MQC_E_LIMIT;
  }
}

template <typename... A>
int dispatch_conv(int dtype, A... args) {
  switch (dtype) {
    case MQC_F32: return launch_conv<float>(args...);
    case MQC_BF16: return launch_conv<bf16_t>(args...);
    case MQC_F16: return launch_conv<f16_t>(args...);
    default: return MQC_E_DTYPE;
  }
}

template <typename T, int K>
int launch_conv_step_k(const void* x, int64_t xs, void* tail, const float* w, const float* bias,
                       void* out, int64_t Bn, int64_t C, hipStream_t s) {
  const int64_t blocks = (Bn * C + kConvThreads - 1) / kConvThreads;
  if (blocks > 0x7fffffffLL) return MQC_E_LIMIT;
  // The forward's rounding for a sequence of this width (its 16-byte path
  // applies when C is a multiple of the vector width).
  if (C % conv_vec<T>() == 0)
    conv_silu_step_kernel<T, K, true><<<dim3((unsigned)blocks), dim3(kConvThreads), 0, s>>>(
        (const T*)x, xs, (T*)tail, w, bias, (T*)out, Bn, C);
  else
    conv_silu_step_kernel<T, K, false><<<dim3((unsigned)blocks), dim3(kConvThreads), 0, s>>>(
        (const T*)x, xs, (T*)tail, w, bias, (T*)out, Bn, C);
  return launch_status();
}

template <typename T>
int launch_conv_step(const void* x, int64_t xs, void* tail, const float* w, const float* bias,
                     void* out, int64_t Bn, int64_t C, int64_t K, hipStream_t s) {
  if (Bn == 0 || C == 0) return MQC_OK;
  if (!aligned(x, sizeof(T)) || !aligned(out, sizeof(T)) || !aligned(tail, sizeof(T)) ||
      !aligned(w, 4) || (bias && !aligned(bias, 4)))
    return MQC_E_ALIGN;
  switch (K) {
    case 1: return launch_conv_step_k<T, 1>(x, xs, tail, w, bias, out, Bn, C, s);
    case 2: return launch_conv_step_k<T, 2>(x, xs, tail, w, bias, out, Bn, C, s);
    case 3: return launch_conv_step_k<T, 3>(x, xs, tail, w, bias, out, Bn, C, s);
    case 4: return launch_conv_step_k<T, 4>(x, xs, tail, w, bias, out, Bn, C, s);
    case 5: return launch_conv_step_k<T, 5>(x, xs, tail, w, bias, out, Bn, C, s);
    case 6: return launch_conv_step_k<T, 6>(x, xs, tail, w, bias, out, Bn, C, s);
    case 7: return launch_conv_step_k<T, 7>(x, xs, tail, w, bias, out, Bn, C, s);
    case 8: return launch_conv_step_k<T, 8>(x, xs, tail, w, bias, out, Bn, C, s);
    default: return MQC_E_LIMIT;
  }
}

}  // namespace mqc

using namespace mqc;

extern "C" {

int mqc_conv_run_length(void) { return kConvRun; }

int mqc_causal_conv_silu_fwd(const void* x, int64_t x_row_stride, const float* w, const float* bias,
                             void* out, int64_t batch, int64_t seq_len, int64_t channels,
                             int64_t kernel, int dtype, void* stream) {
  if (batch < 0 || seq_len < 0 || channels < 0 || kernel < 1 || x_row_stride < channels)
    return MQC_E_SHAPE;
  if (kernel > kConvMaxK) return MQC_E_LIMIT;
  if (batch > 0 && seq_len > 0 && channels > 0 && (!x || !w || !out)) return MQC_E_NULL;
  return dispatch_conv(dtype, false, x, x_row_stride, w, bias, (const void*)nullptr, out,
                       (int64_t)0, (float*)nullptr, (float*)nullptr, batch, seq_len, channels,
                       kernel, (hipStream_t)stream);
}

int mqc_causal_conv_silu_bwd(const void* x, int64_t x_row_stride, const float* w,
                             const float* bias, const void* gout, void* dx, int64_t dx_row_stride,
                             float* dw_part, float* dbias_part, int64_t batch, int64_t seq_len,
                             int64_t channels, int64_t kernel, int dtype, void* stream) {
  if (batch < 0 || seq_len < 0 || channels < 0 || kernel < 1 || x_row_stride < channels ||
      dx_row_stride < channels)
    return MQC_E_SHAPE;
  if (kernel > kConvMaxK) return MQC_E_LIMIT;
  if (batch > 0 && seq_len > 0 && channels > 0 &&
      (!x || !w || !gout || !dx || !dw_part || !dbias_part))
    return MQC_E_NULL;
  return dispatch_conv(dtype, true, x, x_row_stride, w, bias, gout, dx, dx_row_stride, dw_part,
                       dbias_part, batch, seq_len, channels, kernel, (hipStream_t)stream);
}

int mqc_causal_conv_silu_step(const void* x, int64_t x_row_stride, void* tail, const float* w,
                              const float* bias, void* out, int64_t batch, int64_t channels,
                              int64_t kernel, int dtype, void* stream) {
  if (batch < 0 || channels < 0 || kernel < 1 || x_row_stride < channels) return MQC_E_SHAPE;
  if (kernel > kConvMaxK) return MQC_E_LIMIT;
  if (batch > 0 && channels > 0 && (!x || !w || !out || (kernel > 1 && !tail)))
    return MQC_E_NULL;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MQC_F32: return launch_conv_step<float>(x, x_row_stride, tail, w, bias, out, batch, channels, kernel, s);
    case MQC_BF16: return launch_conv_step<bf16_t>(x, x_row_stride, tail, w, bias, out, batch, channels, kernel, s);
    case MQC_F16: return launch_conv_step<f16_t>(x, x_row_stride, tail, w, bias, out, batch, channels, kernel, s);
    default: return MQC_E_DTYPE;
  }
}

}  // extern "C"
