// Quaternion LayerNorm (mambaqc/kernels/quaternion_norm.py:219-245):
//   n_i   = sqrt(|q_i|^2 + eps)
//   mu    = mean_i n_i,   var = mean_i (n_i - mu)^2      (biased)
//   out_i = gamma_i * (n_i - mu) / sqrt(var + eps) * q_i / (n_i + eps) + beta_i
//
// One row of d quaternions per wavefront (WPR = 1) or per workgroup of WPR
// wavefronts. The row is read once into registers (lane L holds quaternions
// L, L+64*WPR, ...), the two statistics are exact two-pass reductions over
// those registers (cross-lane butterfly, then LDS across the wavefronts of a
// workgroup), and the row is written once: one HBM read and one write per
// element. Masked tail lanes contribute nothing to the sums, so the
// statistics are over exactly d norms for any d.
#include "common.hpp"

namespace mqc {

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

template <int WPR>
__device__ inline float row_sum(float v, float* red) {
  v = wave_sum(v);
  if constexpr (WPR == 1) {
    return v;
  } else {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < WPR; ++i) s += red[i];
    return s;
  }
}

// NPL: quaternions per lane (register capacity); rows of d <= NPL*64*WPR.
template <typename T, int NPL, int WPR>
__global__ __launch_bounds__(256) void qln_kernel(const T* __restrict__ q,
                                                  const float* __restrict__ gamma,
                                                  const float* __restrict__ beta,
                                                  T* __restrict__ out, float* __restrict__ mean_out,
                                                  float* __restrict__ rstd_out, int64_t rows,
                                                  int64_t d, float eps) {
  constexpr int RPB = 4 / WPR;  // rows per 256-thread block
  __shared__ float red[RPB][WPR > 1 ? WPR : 1];
  const int tid = threadIdx.x;
  const int sub = tid / (64 * WPR);        // row slot inside the block
  const int t = tid - sub * 64 * WPR;      // thread index inside the row
  const int64_t row = (int64_t)blockIdx.x * RPB + sub;
  const bool rvalid = row < rows;
  constexpr int TPR = 64 * WPR;
  // Rows and elements past the end are clamped onto valid addresses (and their
  // values masked), so the NPL loads carry no predicate and issue back to back.
  const T* qr = q + (rvalid ? row : rows - 1) * d * 4;

  float v[NPL][4];
  float n[NPL];
#pragma unroll
  for (int m = 0; m < NPL; ++m) {
    const int64_t i = t + (int64_t)m * TPR;
    load_vec<T, 4>(qr + (i < d ? i : d - 1) * 4, v[m]);
  }
#pragma unroll
  for (int m = 0; m < NPL; ++m) {
    const bool in = t + (int64_t)m * TPR < d;
#pragma unroll
    for (int c = 0; c < 4; ++c) v[m][c] = in ? v[m][c] : 0.f;
  }
  float s1 = 0.f;
#pragma unroll
  for (int m = 0; m < NPL; ++m) {
    const bool in = t + (int64_t)m * TPR < d;
    n[m] = sqrtf(v[m][0] * v[m][0] + v[m][1] * v[m][1] + v[m][2] * v[m][2] + v[m][3] * v[m][3] + eps);
    s1 += in ? n[m] : 0.f;
  }
  const float inv_d = 1.f / (float)d;
  const float mu = row_sum<WPR>(s1, red[sub]) * inv_d;
  float s2 = 0.f;
#pragma unroll
  for (int m = 0; m < NPL; ++m) {
    const bool in = t + (int64_t)m * TPR < d;
    const float c = n[m] - mu;
    s2 = in ? fmaf(c, c, s2) : s2;
  }
  const float var = row_sum<WPR>(s2, red[sub]) * inv_d;
  const float rstd = 1.f / sqrtf(var + eps);

  if (rvalid) {
    if (t == 0) {
      if (mean_out) mean_out[row] = mu;
      if (rstd_out) rstd_out[row] = rstd;
    }
    T* orow = out + row * d * 4;
#pragma unroll
    for (int m = 0; m < NPL; ++m) {
      const int64_t i = t + (int64_t)m * TPR;
      const int64_t ic = i < d ? i : d - 1;
      const float f = gamma[ic] * ((n[m] - mu) * rstd) / (n[m] + eps);
      const float4 bt = reinterpret_cast<const float4*>(beta)[ic];
      float o[4] = {fmaf(f, v[m][0], bt.x), fmaf(f, v[m][1], bt.y), fmaf(f, v[m][2], bt.z),
                    fmaf(f, v[m][3], bt.w)};
      if (i < d) store_vec<T, 4>(orow + i * 4, o);
    }
  }
}

template <typename T, int NPL, int WPR>
int launch_qln_n(const void* q, const float* gamma, const float* beta, void* out, float* mean,
                 float* rstd, int64_t rows, int64_t d, float eps, hipStream_t s) {
  constexpr int RPB = 4 / WPR;
  const int64_t blocks = (rows + RPB - 1) / RPB;
  if (blocks > 0x7fffffffLL) return MQC_E_LIMIT;
  qln_kernel<T, NPL, WPR><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
      (const T*)q, gamma, beta, (T*)out, mean, rstd, rows, d, eps);
  return launch_status();
}

template <typename T>
int launch_qln(const void* q, const float* gamma, const float* beta, void* out, float* mean,
               float* rstd, int64_t rows, int64_t d, float eps, hipStream_t s) {
  if (rows == 0) return MQC_OK;
  if (d == 0) return MQC_E_SHAPE;
  if (!aligned(q, 4 * sizeof(T)) || !aligned(out, 4 * sizeof(T)) || !aligned(beta, 16) ||
      !aligned(gamma, 4))
    return MQC_E_ALIGN;
#define MQC_QLN(NPL, WPR)                                                   \
  if (d <= (int64_t)(NPL) * 64 * (WPR))                                     \
    return launch_qln_n<T, NPL, WPR>(q, gamma, beta, out, mean, rstd, rows, d, eps, s);
  MQC_QLN(1, 1)
  MQC_QLN(2, 1)
  MQC_QLN(4, 1)
  MQC_QLN(2, 4)
  MQC_QLN(4, 4)
  MQC_QLN(6, 4)
  MQC_QLN(8, 4)
  MQC_QLN(16, 4)
  MQC_QLN(32, 4)
#undef MQC_QLN
  return MQC_E_LIMIT;
}

// ---------------------------------------------------------------------------
// Backward. With n-hat = (n - mu) * rstd, dir = q / (n + eps), out = gamma n-hat dir + beta
// and e_i = <dout_i, dir_i>:
//   dbeta_i  = sum_rows dout_i,   dgamma_i = sum_rows n-hat_i e_i
//   dn-hat_i = gamma_i e_i
//   dn_i     = -gamma_i n-hat_i e_i / (n_i + eps)
//              + rstd (dn-hat_i - mean(dn-hat) - n-hat_i mean(dn-hat n-hat))
//   dq_i     = gamma_i n-hat_i / (n_i + eps) * dout_i + dn_i / n_i * q_i
// The kernel writes dq and ne_i = n-hat_i e_i per (row, i) (fp32); the caller
// sums ne and dout over rows for dgamma and dbeta. mu and rstd are the
// forward's saved statistics.
// ---------------------------------------------------------------------------
template <typename T, int NPL, int WPR>
__global__ __launch_bounds__(256) void qln_bwd_kernel(const T* __restrict__ q,
                                                      const T* __restrict__ dout,
                                                      const float* __restrict__ gamma,
                                                      const float* __restrict__ mean,
                                                      const float* __restrict__ rstd_in,
                                                      T* __restrict__ dq, float* __restrict__ ne,
                                                      int64_t rows, int64_t d, float eps) {
  constexpr int RPB = 4 / WPR;
  __shared__ float red[RPB][WPR > 1 ? WPR : 1];
  const int tid = threadIdx.x;
  const int sub = tid / (64 * WPR);
  const int t = tid - sub * 64 * WPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + sub;
  const bool rvalid = row < rows;
  constexpr int TPR = 64 * WPR;
  // Clamped rows and elements (values masked) keep the loads unpredicated.
  const int64_t r = rvalid ? row : rows - 1;
  const T* qr = q + r * d * 4;
  const T* gr = dout + r * d * 4;
  const float mu = mean[r];
  const float rstd = rstd_in[r];

  float v[NPL][4], g[NPL][4];
  float nh[NPL], e[NPL], inv_ne[NPL];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int m = 0; m < NPL; ++m) {
    const int64_t i = t + (int64_t)m * TPR;
    const int64_t ic = i < d ? i : d - 1;
    load_vec<T, 4>(qr + ic * 4, v[m]);
    load_vec<T, 4>(gr + ic * 4, g[m]);
  }
#pragma unroll
  for (int m = 0; m < NPL; ++m) {
    const bool in = t + (int64_t)m * TPR < d;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      v[m][c] = in ? v[m][c] : 0.f;
      g[m][c] = in ? g[m][c] : 0.f;
    }
  }
#pragma unroll
  for (int m = 0; m < NPL; ++m) {
    const int64_t i = t + (int64_t)m * TPR;
    const bool in = i < d;
    const float n = sqrtf(v[m][0] * v[m][0] + v[m][1] * v[m][1] + v[m][2] * v[m][2] +
                          v[m][3] * v[m][3] + eps);
    inv_ne[m] = 1.f / (n + eps);
    nh[m] = (n - mu) * rstd;
    e[m] = (g[m][0] * v[m][0] + g[m][1] * v[m][1] + g[m][2] * v[m][2] + g[m][3] * v[m][3]) *
           inv_ne[m];
    const float gmv = gamma[in ? i : d - 1];
    const float dnh = in ? gmv * e[m] : 0.f;
    s1 += dnh;
    s2 = fmaf(dnh, nh[m], s2);
  }
  const float inv_d = 1.f / (float)d;
  const float m1 = row_sum<WPR>(s1, red[sub]) * inv_d;
  const float m2 = row_sum<WPR>(s2, red[sub]) * inv_d;
  if (!rvalid) return;
  T* dqr = dq + row * d * 4;
  float* ner = ne + row * d;
#pragma unroll
  for (int m = 0; m < NPL; ++m) {
    const int64_t i = t + (int64_t)m * TPR;
    const float gm = gamma[i < d ? i : d - 1];
    if (i < d) {
      const float n = sqrtf(v[m][0] * v[m][0] + v[m][1] * v[m][1] + v[m][2] * v[m][2] +
                            v[m][3] * v[m][3] + eps);
      const float a = gm * nh[m] * inv_ne[m];                 // coefficient of dout
      const float dn = -a * e[m] + rstd * (gm * e[m] - m1 - nh[m] * m2);
      const float bq = dn / n;                                 // coefficient of q
      float o[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = fmaf(a, g[m][c], bq * v[m][c]);
      store_vec<T, 4>(dqr + i * 4, o);
      ner[i] = nh[m] * e[m];
    }
  }
}

template <typename T, int NPL, int WPR>
int launch_qln_bwd_n(const void* q, const void* dout, const float* gamma, const float* mean,
                     const float* rstd, void* dq, float* ne, int64_t rows, int64_t d, float eps,
                     hipStream_t s) {
  constexpr int RPB = 4 / WPR;
  const int64_t blocks = (rows + RPB - 1) / RPB;
  if (blocks > 0x7fffffffLL) return MQC_E_LIMIT;
  qln_bwd_kernel<T, NPL, WPR><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
      (const T*)q, (const T*)dout, gamma, mean, rstd, (T*)dq, ne, rows, d, eps);
  return launch_status();
}

template <typename T>
int launch_qln_bwd(const void* q, const void* dout, const float* gamma, const float* mean,
                   const float* rstd, void* dq, float* ne, int64_t rows, int64_t d, float eps,
                   hipStream_t s) {
  if (rows == 0) return MQC_OK;
  if (d == 0) return MQC_E_SHAPE;
  if (!aligned(q, 4 * sizeof(T)) || !aligned(dout, 4 * sizeof(T)) || !aligned(dq, 4 * sizeof(T)) ||
      !aligned(gamma, 4) || !aligned(mean, 4) || !aligned(rstd, 4) || !aligned(ne, 4))
    return MQC_E_ALIGN;
#define MQC_QLNB(NPL, WPR)                                                        \
  if (d <= (int64_t)(NPL) * 64 * (WPR))                                           \
    return launch_qln_bwd_n<T, NPL, WPR>(q, dout, gamma, mean, rstd, dq, ne, rows, d, eps, s);
  MQC_QLNB(1, 1)
  MQC_QLNB(2, 1)
  MQC_QLNB(4, 1)
  MQC_QLNB(8, 1)
  MQC_QLNB(6, 4)
  MQC_QLNB(8, 4)
  MQC_QLNB(16, 4)
  MQC_QLNB(32, 4)
#undef MQC_QLNB
  return MQC_E_LIMIT;
}

}  // namespace mqc

using namespace mqc;

extern "C" int mqc_qln_fwd(const void* q, const float* gamma, const float* beta, void* out,
                           float* mean, float* rstd, int64_t rows, int64_t d, float eps,
                           int dtype, void* stream) {
  if (rows < 0 || d < 0) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  if (rows > 0 && (!q || !gamma || !beta || !out)) return MQC_E_NULL;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MQC_F32: return launch_qln<float>(q, gamma, beta, out, mean, rstd, rows, d, eps, s);
    case MQC_BF16: return launch_qln<bf16_t>(q, gamma, beta, out, mean, rstd, rows, d, eps, s);
    default: return launch_qln<f16_t>(q, gamma, beta, out, mean, rstd, rows, d, eps, s);
  }
}

extern "C" int mqc_qln_bwd(const void* q, const void* dout, const float* gamma, const float* mean,
                           const float* rstd, void* dq, float* ne, int64_t rows, int64_t d,
                           float eps, int dtype, void* stream) {
  if (rows < 0 || d < 0) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  if (rows > 0 && (!q || !dout || !gamma || !mean || !rstd || !dq || !ne)) return MQC_E_NULL;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MQC_F32: return launch_qln_bwd<float>(q, dout, gamma, mean, rstd, dq, ne, rows, d, eps, s);
    case MQC_BF16: return launch_qln_bwd<bf16_t>(q, dout, gamma, mean, rstd, dq, ne, rows, d, eps, s);
    default: return launch_qln_bwd<f16_t>(q, dout, gamma, mean, rstd, dq, ne, rows, d, eps, s);
  }
}
