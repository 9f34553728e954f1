// Inclusive left-ordered cumulative Hamilton product along the sequence axis:
//   out[b,t,l] = q[b,t,l] (x) out[b,t-1,l]        (out[b,-1,l] = 1)
// (semantics of mambaqc/kernels/parallel_scan.py:267-295).
//
// Layout: q and out are [batch, seq_len, lanes, 4] row-major, so for a fixed
// (b, t) the `lanes` quaternions are contiguous. A workgroup owns one batch
// row b and a block of 64 lanes; its 64 threads per wave sit on consecutive
// lanes (one fully coalesced 1 KiB fp32 row segment per step). The W waves of
// the workgroup split the time axis: in each tile of W*TW steps, wave w walks
// steps [w*TW, (w+1)*TW) from the identity, keeping its TW local prefixes in
// registers. The W wave aggregates meet in LDS, where each wave forms its
// exclusive carry
//     E_w = A_{w-1} (x) ... (x) A_0 (x) carry
// with the later aggregate always on the LEFT (the monoid is
// non-commutative), then multiplies its local prefixes by E_w on the right
// and stores. Every element is read once and written once.
#include "common.hpp"

namespace mqc {

template <typename T, int W, int TW>
__global__ __launch_bounds__(W * 64) void cumprod_scan_kernel(const T* __restrict__ q,
                                                              T* __restrict__ out, int64_t T_len,
                                                              int64_t L) {
  __shared__ float4 agg[W][64];
  __shared__ float4 carry[64];

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int64_t l = (int64_t)blockIdx.x * 64 + lane;
  const int64_t b = blockIdx.y;
  const bool valid = l < L;
  const int64_t row = L * 4;  // elements per (b, t)
  // Lanes past L and steps past T load from clamped (valid) addresses and use
  // the identity instead, so the loads carry no predicate and issue together.
  const T* qb = q + b * T_len * row + (valid ? l : L - 1) * 4;
  T* ob = out + b * T_len * row + l * 4;

  if (w == 0) carry[lane] = make_float4(1.f, 0.f, 0.f, 0.f);

  for (int64_t tile = 0; tile < T_len; tile += (int64_t)W * TW) {
    const int64_t t0 = tile + (int64_t)w * TW;
    int64_t left = T_len - t0;
    const int n = left <= 0 ? 0 : (left >= TW ? TW : (int)left);

    quat v[TW];
#pragma unroll
    for (int j = 0; j < TW; ++j) {
      int64_t tj = t0 + j;
      tj = tj < T_len ? tj : T_len - 1;
      float e[4];
      load_vec<T, 4>(qb + tj * row, e);
      const bool use = valid && j < n;
      v[j] = use ? quat_from(e) : quat{1.f, 0.f, 0.f, 0.f};
    }
    // Local inclusive prefixes: v[j] <- q_j (x) v[j-1].
#pragma unroll
    for (int j = 1; j < TW; ++j) v[j] = qmul(v[j], v[j - 1]);

    agg[w][lane] = make_float4(v[TW - 1].w, v[TW - 1].x, v[TW - 1].y, v[TW - 1].z);
    __syncthreads();

    float4 c = carry[lane];
    quat E{c.x, c.y, c.z, c.w};
    for (int u = 0; u < w; ++u) {
      float4 a = agg[u][lane];
      E = qmul(quat{a.x, a.y, a.z, a.w}, E);
    }

    if (valid) {
#pragma unroll
      for (int j = 0; j < TW; ++j) {
        if (j < n) {
          quat r = qmul(v[j], E);
          float e[4] = {r.w, r.x, r.y, r.z};
          store_vec<T, 4, true>(ob + (t0 + j) * row, e);
        }
      }
    }
    __syncthreads();  // all waves have read carry and agg
    if (w == W - 1) {
      quat r = qmul(v[TW - 1], E);
      carry[lane] = make_float4(r.w, r.x, r.y, r.z);
    }
    __syncthreads();
  }
}

template <typename T>
int launch_cumprod(const void* q, void* out, int64_t B, int64_t T_len, int64_t L, hipStream_t s) {
  if (B == 0 || T_len == 0 || L == 0) return MQC_OK;
  if (!aligned(q, 4 * sizeof(T)) || !aligned(out, 4 * sizeof(T))) return MQC_E_ALIGN;
  if (B > 65535) return MQC_E_LIMIT;
  constexpr int W = 4, TW = 16;
  dim3 grid((unsigned)((L + 63) / 64), (unsigned)B);
  cumprod_scan_kernel<T, W, TW><<<grid, dim3(W * 64), 0, s>>>((const T*)q, (T*)out, T_len, L);
  return launch_status();
}

}  // namespace mqc

using namespace mqc;

extern "C" int mqc_cumprod_scan_fwd(const void* q, void* out, int64_t batch, int64_t seq_len,
                                    int64_t lanes, int dtype, void* stream) {
  if (batch < 0 || seq_len < 0 || lanes < 0) return MQC_E_SHAPE;
  if (batch > 0 && seq_len > 0 && lanes > 0 && (!q || !out)) return MQC_E_NULL;
  if (lanes > ((int64_t)1 << 37)) return MQC_E_LIMIT;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case MQC_F32: return launch_cumprod<float>(q, out, batch, seq_len, lanes, s);
    case MQC_BF16: return launch_cumprod<bf16_t>(q, out, batch, seq_len, lanes, s);
    case MQC_F16: return launch_cumprod<f16_t>(q, out, batch, seq_len, lanes, s);
    default: return MQC_E_DTYPE;
  }
}
