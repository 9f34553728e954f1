// Quaternion selective-state-space recurrence, fused.
//
//   h_t = q_t (x) h_{t-1} + B_t (x) S_t        (S broadcast over d_state)
//   y_t = sum_k C_{t,k} (x) h_{t,k} + D_t * S_t
//
// (mambaqc/kernels/ssm_fused.py:363-379 and :405-430.)
//
// Two operand forms share one kernel:
//   MODE_DL  the block's form: q_t = Cayley(delta_t * Lambda) is computed in
//            registers from a per-(d,k) Lambda (closed form below), S = (s,0,0,0)
//            so B (x) S = s * B, and D is a per-d vector. Neither z nor q is
//            ever written to memory (quaternion_mamba2_block.py:183-228).
//   MODE_Q   q, S (full quaternion) and D (strided [B,T,D]) given explicitly,
//            as in ssm_forward_fused / ssm_step_fused.
//
// Work decomposition. Every (b, d, k) is an independent sequential recurrence
// over t. A group of G consecutive lanes owns one (b, d); lane j of the group
// owns KPL consecutive k (so one lane reads KPL*4 contiguous elements of B and
// of C per step, 16 bytes for bf16 with KPL = 2). Each lane walks all T steps,
// keeping its KPL states in registers, with a ring of PF steps of operands in
// flight (raw loaded bits; they are unpacked only when consumed, so the loads
// of step t+PF overlap the arithmetic of step t). The per-step sum over k is
// an in-register FMA chain across the lane's KPL states followed by a G-lane
// transpose-reduce: the first two butterfly stages swap half of the four
// components with the partner lane instead of reducing all four, so after
// them each lane carries one component and the remaining log2(G)-2 stages are
// single adds.
//
// Cayley closed form. For z = (a, v), den = 1 - z/2, num = 1 + z/2:
//   den^-1 (x) num = (1 - |z|^2/4, v) / max(|den|^2, eps),
//   |den|^2 = 1 - a + |z|^2/4,
// because conj(den) and num share v's axis and therefore commute. With
// z = delta * Lambda and n2 = |Lambda|^2 / 4 per (d, k):
//   N = max(1 - delta*a_L + delta^2 n2, eps),
//   q = ((1 - delta^2 n2) / N, delta * v_L / N),
// one reciprocal per (t, d, k).
#include <type_traits>

#include "common.hpp"

namespace mqc {

constexpr int MODE_DL = 0;
constexpr int MODE_Q = 1;
constexpr int kSsmThreads = 256;

// Raw bits of N consecutive storage elements (unpacked only on use).
template <typename T, int N>
struct Raw {
  static constexpr int W = (N * (int)sizeof(T) + 3) / 4;
  uint32_t w[W];
};

template <typename T, int N>
__device__ inline void raw_load(const T* __restrict__ p, Raw<T, N>& r) {
  constexpr int W = Raw<T, N>::W;
  constexpr int bytes = N * (int)sizeof(T);
  if constexpr (bytes % 16 == 0) {
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      uint4 v = reinterpret_cast<const uint4*>(p)[i];
      r.w[4 * i + 0] = v.x;
      r.w[4 * i + 1] = v.y;
      r.w[4 * i + 2] = v.z;
      r.w[4 * i + 3] = v.w;
    }
  } else if constexpr (bytes == 8) {
    uint2 v = *reinterpret_cast<const uint2*>(p);
    r.w[0] = v.x;
    r.w[1] = v.y;
  } else if constexpr (bytes == 4) {
    r.w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else {
    static_assert(bytes == 2, "unsupported raw width");
    r.w[0] = *reinterpret_cast<const uint16_t*>(p);
  }
}

template <typename T, int N>
__device__ inline float raw_get(const Raw<T, N>& r, int e) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(r.w[e]);
  } else if constexpr (std::is_same<T, bf16_t>::value) {
    const uint32_t word = r.w[e >> 1];
    return __uint_as_float((e & 1) ? (word & 0xffff0000u) : (word << 16));
  } else {
    const uint32_t word = r.w[e >> 1];
    return io<T>::bits_to_f32((e & 1) ? (word >> 16) : (word & 0xffffu));
  }
}

template <typename T, int N>
__device__ inline quat raw_quat(const Raw<T, N>& r, int qi) {
  return quat{raw_get(r, 4 * qi + 0), raw_get(r, 4 * qi + 1), raw_get(r, 4 * qi + 2),
              raw_get(r, 4 * qi + 3)};
}

struct SsmArgs {
  // MODE_DL: delta, s [B,T,D]; lam_alpha [D,S]; lam_imag [D,S,3]; dvec [D]
  const void* delta;
  const void* s;
  const float* lam_alpha;
  const float* lam_imag;
  const float* dvec;
  // MODE_Q: q [B,T,D,S,4]; Sq [B,T,D,4]; Dq strided [B,T,D]
  const void* q;
  const void* Sq;
  const void* Dq;
  int64_t d_sb, d_st, d_sd;
  // both
  const void* Bm;
  const void* Cm;
  const void* h0;
  void* y;
  void* h_last;
  int64_t batch, T, Dm, S;
  float eps;
};

template <typename T, int MODE, int KPL>
struct Step;

template <typename T, int KPL>
struct Step<T, MODE_DL, KPL> {
  Raw<T, 1> delta, s;
  Raw<T, 4 * KPL> B, C;
};

template <typename T, int KPL>
struct Step<T, MODE_Q, KPL> {
  Raw<T, 4 * KPL> q, B, C;
  Raw<T, 4> S;
  Raw<T, 1> D;
};

// Sum `acc` over the G lanes of a group (G a power of two, groups aligned in
// the wave). Returns, in v[0..NC), the components this lane ends up holding,
// and the index of the first of them in c0 (they are consecutive).
//   G == 1: all four, G == 2: two, G >= 4: one.
template <int G>
__device__ inline int group_reduce(const quat& acc, int lane, float (&v)[4], int& c0) {
  if constexpr (G == 1) {
    v[0] = acc.w; v[1] = acc.x; v[2] = acc.y; v[3] = acc.z;
    c0 = 0;
    return 4;
  } else {
    const bool odd = lane & 1;
    // Stage xor-1: even lanes keep components (0,1), odd lanes keep (2,3),
    // each sends the other pair to its partner.
    const float s0 = odd ? acc.w : acc.y;
    const float s1 = odd ? acc.x : acc.z;
    float k0 = odd ? acc.y : acc.w;
    float k1 = odd ? acc.z : acc.x;
    k0 += __shfl_xor(s0, 1);
    k1 += __shfl_xor(s1, 1);
    if constexpr (G == 2) {
      v[0] = k0; v[1] = k1;
      c0 = odd ? 2 : 0;
      return 2;
    } else {
      // Stage xor-2: lanes with bit 1 clear keep the first of the pair.
      const bool hi = lane & 2;
      const float snd = hi ? k0 : k1;
      float kk = hi ? k1 : k0;
      kk += __shfl_xor(snd, 2);
#pragma unroll
      for (int m = 4; m < G; m <<= 1) kk += __shfl_xor(kk, m);
      v[0] = kk;
      c0 = (odd ? 2 : 0) + (hi ? 1 : 0);
      return 1;
    }
  }
}

__device__ inline float softplus_f(float x) {
  // torch.nn.functional.softplus with beta = 1, threshold = 20.
  return x > 20.f ? x : log1pf(expf(x));
}

template <typename T, int MODE, int KPL, int G, int PF>
__global__ __launch_bounds__(kSsmThreads) void ssm_scan_kernel(SsmArgs a) {
  static_assert((G & (G - 1)) == 0 && G <= 64, "G must be a power of two <= 64");
  const int lane = threadIdx.x & 63;
  const int64_t gi = (int64_t)blockIdx.x * kSsmThreads + threadIdx.x;
  const int64_t grp = gi / G;
  const int j = (int)(gi & (G - 1));
  const int64_t n_groups = a.batch * a.Dm;
  const bool gvalid = grp < n_groups;
  const int k0 = j * KPL;
  const bool active = gvalid && k0 < a.S;
  const int64_t b = gvalid ? grp / a.Dm : 0;
  const int64_t d = gvalid ? grp - b * a.Dm : 0;

  const int64_t step_bc = a.Dm * a.S * 4;          // elements per t in B, C, q
  const int64_t base_bc = (b * a.T * a.Dm + d) * a.S * 4 + (int64_t)k0 * 4;
  const int64_t step_tok = a.Dm;                   // elements per t in delta, s
  const int64_t base_tok = b * a.T * a.Dm + d;

  const T* Bp = (const T*)a.Bm + base_bc;
  const T* Cp = (const T*)a.Cm + base_bc;

  // Per-(d,k) constants of the Cayley closed form (MODE_DL).
  float la[KPL], ln2[KPL], lv[KPL][3];
  if constexpr (MODE == MODE_DL) {
#pragma unroll
    for (int kk = 0; kk < KPL; ++kk) {
      la[kk] = 0.f; ln2[kk] = 0.f; lv[kk][0] = lv[kk][1] = lv[kk][2] = 0.f;
      if (active) {
        const int64_t dk = d * a.S + k0 + kk;
        const float ar = -softplus_f(a.lam_alpha[dk]);
        const float v0 = tanhf(a.lam_imag[dk * 3 + 0]);
        const float v1 = tanhf(a.lam_imag[dk * 3 + 1]);
        const float v2 = tanhf(a.lam_imag[dk * 3 + 2]);
        la[kk] = ar;
        ln2[kk] = 0.25f * (ar * ar + v0 * v0 + v1 * v1 + v2 * v2);
        lv[kk][0] = v0; lv[kk][1] = v1; lv[kk][2] = v2;
      }
    }
  }
  const float dskip = (MODE == MODE_DL && gvalid) ? a.dvec[d] : 0.f;

  // States.
  quat h[KPL];
#pragma unroll
  for (int kk = 0; kk < KPL; ++kk) h[kk] = quat{0.f, 0.f, 0.f, 0.f};
  if (a.h0 && active) {
    float e[4 * KPL];
    load_vec<T, 4 * KPL>((const T*)a.h0 + ((b * a.Dm + d) * a.S + k0) * 4, e);
#pragma unroll
    for (int kk = 0; kk < KPL; ++kk) h[kk] = quat_from(&e[4 * kk]);
  }

  Step<T, MODE, KPL> ring[PF];
  auto load_step = [&](Step<T, MODE, KPL>& st, int64_t t) {
    if constexpr (MODE == MODE_DL) {
      if (gvalid) {
        raw_load<T, 1>((const T*)a.delta + base_tok + t * step_tok, st.delta);
        raw_load<T, 1>((const T*)a.s + base_tok + t * step_tok, st.s);
      }
    } else {
      if (gvalid) {
        raw_load<T, 4>((const T*)a.Sq + (base_tok + t * step_tok) * 4, st.S);
        raw_load<T, 1>((const T*)a.Dq + b * a.d_sb + t * a.d_st + d * a.d_sd, st.D);
      }
      if (active) raw_load<T, 4 * KPL>((const T*)a.q + base_bc + t * step_bc, st.q);
    }
    if (active) {
      raw_load<T, 4 * KPL>(Bp + t * step_bc, st.B);
      raw_load<T, 4 * KPL>(Cp + t * step_bc, st.C);
    }
  };

  // Inactive lanes never load: their operands stay zero, so they add nothing.
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    Step<T, MODE, KPL>& st = ring[i];
    if constexpr (MODE == MODE_DL) {
      st.delta.w[0] = 0; st.s.w[0] = 0;
    } else {
#pragma unroll
      for (int e = 0; e < Raw<T, 4 * KPL>::W; ++e) st.q.w[e] = 0;
#pragma unroll
      for (int e = 0; e < Raw<T, 4>::W; ++e) st.S.w[e] = 0;
      st.D.w[0] = 0;
    }
#pragma unroll
    for (int e = 0; e < Raw<T, 4 * KPL>::W; ++e) { st.B.w[e] = 0; st.C.w[e] = 0; }
  }

  const int64_t Tn = a.T;
  const int64_t t_last = Tn - 1;
#pragma unroll
  for (int i = 0; i < PF; ++i) load_step(ring[i], i < Tn ? i : t_last);

  T* yp = (T*)a.y + base_tok * 4;
  const int64_t step_y = a.Dm * 4;

  for (int64_t t0 = 0; t0 < Tn; t0 += PF) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int64_t t = t0 + i;
      if (t >= Tn) break;
      const Step<T, MODE, KPL> cur = ring[i];
      // Refill this slot with step t + PF (clamped: the tail re-reads the
      // last step, which keeps the loads branch-free).
      {
        const int64_t tn = t + PF;
        load_step(ring[i], tn < Tn ? tn : t_last);
      }

      quat acc{0.f, 0.f, 0.f, 0.f};
      float sv = 0.f;
      float Sv[4] = {0.f, 0.f, 0.f, 0.f};
      if constexpr (MODE == MODE_DL) {
        const float dl = raw_get(cur.delta, 0);
        sv = raw_get(cur.s, 0);
        const float dl2 = dl * dl;
#pragma unroll
        for (int kk = 0; kk < KPL; ++kk) {
          float N = fmaf(dl2, ln2[kk], fmaf(-dl, la[kk], 1.f));
          N = fmaxf(N, a.eps);
          const float r = __builtin_amdgcn_rcpf(N);
          const float c = dl * r;
          const quat qd{fmaf(-dl2, ln2[kk], 1.f) * r, c * lv[kk][0], c * lv[kk][1],
                        c * lv[kk][2]};
          const quat Bk = raw_quat(cur.B, kk);
          quat hn{sv * Bk.w, sv * Bk.x, sv * Bk.y, sv * Bk.z};
          qmul_acc(hn, qd, h[kk]);
          h[kk] = hn;
          qmul_acc(acc, raw_quat(cur.C, kk), hn);
        }
      } else {
        const quat Sq = raw_quat(cur.S, 0);
        Sv[0] = Sq.w; Sv[1] = Sq.x; Sv[2] = Sq.y; Sv[3] = Sq.z;
#pragma unroll
        for (int kk = 0; kk < KPL; ++kk) {
          const quat qk = raw_quat(cur.q, kk);
          quat hn = qmul(raw_quat(cur.B, kk), Sq);
          qmul_acc(hn, qk, h[kk]);
          h[kk] = hn;
          qmul_acc(acc, raw_quat(cur.C, kk), hn);
        }
      }

      float v[4];
      int c0;
      const int nc = group_reduce<G>(acc, lane, v, c0);
      const bool writer = gvalid && (G < 4 || j < 4);
      if (writer) {
        T* yo = yp + t * step_y;
        if constexpr (MODE == MODE_DL) {
          if (c0 == 0) v[0] = fmaf(dskip, sv, v[0]);
        } else {
          const float Dv = raw_get(cur.D, 0);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (e < nc) v[e] = fmaf(Dv, Sv[c0 + e], v[e]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (e < nc) store_scalar(yo + c0 + e, v[e]);
      }
    }
  }

  if (a.h_last && active) {
    float e[4 * KPL];
#pragma unroll
    for (int kk = 0; kk < KPL; ++kk) {
      e[4 * kk + 0] = h[kk].w; e[4 * kk + 1] = h[kk].x;
      e[4 * kk + 2] = h[kk].y; e[4 * kk + 3] = h[kk].z;
    }
    store_vec<T, 4 * KPL>((T*)a.h_last + ((b * a.Dm + d) * a.S + k0) * 4, e);
  }
}

template <typename T, int MODE, int KPL, int G, int PF>
int launch_ssm_g(const SsmArgs& a, hipStream_t s) {
  const int64_t lanes = a.batch * a.Dm * G;
  const int64_t blocks = (lanes + kSsmThreads - 1) / kSsmThreads;
  if (blocks > 0x7fffffffLL) return MQC_E_LIMIT;
  ssm_scan_kernel<T, MODE, KPL, G, PF><<<dim3((unsigned)blocks), dim3(kSsmThreads), 0, s>>>(a);
  return launch_status();
}

template <typename T, int MODE, int KPL>
int launch_ssm_kpl(const SsmArgs& a, hipStream_t s) {
  const int64_t per = a.S / KPL;  // lanes needed per (b, d)
  // Steps of operands in flight per lane; wide lanes hold more bytes per step.
  constexpr int PF = KPL * (int)sizeof(T) >= 8 ? 4 : 8;
  if (per <= 1) return launch_ssm_g<T, MODE, KPL, 1, PF>(a, s);
  if (per <= 2) return launch_ssm_g<T, MODE, KPL, 2, PF>(a, s);
  if (per <= 4) return launch_ssm_g<T, MODE, KPL, 4, PF>(a, s);
  if (per <= 8) return launch_ssm_g<T, MODE, KPL, 8, PF>(a, s);
  if (per <= 16) return launch_ssm_g<T, MODE, KPL, 16, PF>(a, s);
  if (per <= 32) return launch_ssm_g<T, MODE, KPL, 32, PF>(a, s);
  if (per <= 64) return launch_ssm_g<T, MODE, KPL, 64, PF>(a, s);
  return MQC_E_LIMIT;
}

// Lane width: two states per lane gives 16-byte loads of B and C for 16-bit
// storage and a 32-lane reduction at d_state = 64; fp32 keeps one state per
// lane (16-byte loads) unless d_state exceeds 64.
template <typename T, int MODE>
int launch_ssm(const SsmArgs& a, hipStream_t s) {
  if (a.batch == 0 || a.T == 0 || a.Dm == 0) return MQC_OK;
  const uintptr_t qa = 4 * sizeof(T);
  if (!aligned(a.Bm, qa) || !aligned(a.Cm, qa) || !aligned(a.y, sizeof(T)) ||
      (MODE == MODE_Q && (!aligned(a.q, qa) || !aligned(a.Sq, qa))) ||
      (a.h0 && !aligned(a.h0, qa)) || (a.h_last && !aligned(a.h_last, qa)))
    return MQC_E_ALIGN;
  const bool pair_ok = a.S % 2 == 0 && aligned(a.Bm, 16) && aligned(a.Cm, 16) &&
                       (MODE == MODE_DL || aligned(a.q, 16)) && (!a.h0 || aligned(a.h0, 16)) &&
                       (!a.h_last || aligned(a.h_last, 16));
  if constexpr (sizeof(T) == 2) {
    if (pair_ok && a.S <= 128) return launch_ssm_kpl<T, MODE, 2>(a, s);
    if (a.S <= 64) return launch_ssm_kpl<T, MODE, 1>(a, s);
    if (a.S % 4 == 0 && a.S <= 256 && aligned(a.Bm, 16) && aligned(a.Cm, 16))
      return launch_ssm_kpl<T, MODE, 4>(a, s);
    return MQC_E_LIMIT;
  } else {
    if (a.S <= 64) return launch_ssm_kpl<T, MODE, 1>(a, s);
    if (a.S % 2 == 0 && a.S <= 128) return launch_ssm_kpl<T, MODE, 2>(a, s);
    if (a.S % 4 == 0 && a.S <= 256) return launch_ssm_kpl<T, MODE, 4>(a, s);
    return MQC_E_LIMIT;
  }
}

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
  const bool work = batch > 0 && d_inner > 0 && (seq_len > 0 || h_last);
  if (work && d_state > 0 && (!q || !B || !S || !C || !D || !y)) return MQC_E_NULL;
  if (batch > 65535LL * 4096 || d_inner > (1LL << 24) || d_state > 256) return MQC_E_LIMIT;
  SsmArgs a{};
  a.q = q; a.Sq = S; a.Dq = D; a.d_sb = d_sb; a.d_st = d_st; a.d_sd = d_sd;
  a.Bm = B; a.Cm = C; a.h0 = h0; a.y = y; a.h_last = h_last;
  a.batch = batch; a.T = seq_len; a.Dm = d_inner; a.S = d_state; a.eps = 0.f;
  if (seq_len == 0) return MQC_OK;
  return dispatch_ssm<MODE_Q>(a, dtype, (hipStream_t)stream);
}

int mqc_ssm_fused_fwd(const void* delta, const void* s, const void* B, const void* C,
                      const float* lambda_alpha, const float* lambda_imag, const float* D,
                      const void* h0, void* y, void* h_last, int64_t batch, int64_t seq_len,
                      int64_t d_inner, int64_t d_state, float eps, int dtype, void* stream) {
  if (batch < 0 || seq_len < 0 || d_inner < 0 || d_state < 0) return MQC_E_SHAPE;
  if (dtype != MQC_F32 && dtype != MQC_BF16 && dtype != MQC_F16) return MQC_E_DTYPE;
  const bool work = batch > 0 && d_inner > 0 && seq_len > 0;
  if (work && d_state > 0 &&
      (!delta || !s || !B || !C || !lambda_alpha || !lambda_imag || !D || !y))
    return MQC_E_NULL;
  if (batch > 65535LL * 4096 || d_inner > (1LL << 24) || d_state > 256) return MQC_E_LIMIT;
  SsmArgs a{};
  a.delta = delta; a.s = s; a.lam_alpha = lambda_alpha; a.lam_imag = lambda_imag; a.dvec = D;
  a.Bm = B; a.Cm = C; a.h0 = h0; a.y = y; a.h_last = h_last;
  a.batch = batch; a.T = seq_len; a.Dm = d_inner; a.S = d_state; a.eps = eps;
  if (!work) return MQC_OK;
  return dispatch_ssm<MODE_DL>(a, dtype, (hipStream_t)stream);
}

}  // extern "C"
