// Shared device helpers for the mambaqc_amd HIP kernels (gfx950 / CDNA4).
//
// Storage dtypes: fp32, bf16, fp16. All arithmetic is fp32. A quaternion is
// four consecutive elements (w, x, y, z) of the innermost axis, exactly as in
// the reference's [..., 4] tensors (mambaqc/kernels/quaternion_ops.py:259-282).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/mambaqc_hip.h"

namespace mqc {

// ---------------------------------------------------------------------------
// Storage types. bf16 and fp16 are carried as raw 16-bit patterns so that the
// loads below can fetch several of them with one 8- or 16-byte instruction.
// ---------------------------------------------------------------------------
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

template <typename T> struct io;

template <> struct io<float> {
  static constexpr int bytes = 4;
  __device__ static inline float to_f32(float v) { return v; }
  __device__ static inline float from_f32(float v) { return v; }
};

template <> struct io<bf16_t> {
  static constexpr int bytes = 2;
  __device__ static inline float bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }
  __device__ static inline float to_f32(bf16_t v) { return bits_to_f32(v.bits); }
  // Round to nearest even (gfx950's v_cvt_pk_bf16_f32), the rounding torch
  // uses for float -> bfloat16 conversions; NaN stays NaN.
  __device__ static inline bf16_t from_f32(float f) {
    bf16_t r;
    r.bits = __builtin_bit_cast(uint16_t, (__bf16)f);
    return r;
  }
};

template <> struct io<f16_t> {
  static constexpr int bytes = 2;
  __device__ static inline float bits_to_f32(uint32_t b) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)b);
    return (float)h;
  }
  __device__ static inline float to_f32(f16_t v) { return bits_to_f32(v.bits); }
  __device__ static inline f16_t from_f32(float f) {
    _Float16 h = (_Float16)f;
    f16_t r;
    r.bits = __builtin_bit_cast(uint16_t, h);
    return r;
  }
};

// ---------------------------------------------------------------------------
// Vector loads of N consecutive elements (N*bytes is 8 or a multiple of 16)
// into fp32 registers. The pointer must be aligned to min(16, N*bytes).
// ---------------------------------------------------------------------------
template <typename T, int N>
__device__ inline void load_vec(const T* __restrict__ p, float (&out)[N]) {
  if constexpr (sizeof(T) == 4) {
    static_assert(N % 4 == 0, "fp32 loads come in float4 units");
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      float4 v = reinterpret_cast<const float4*>(p)[i];
      out[4 * i + 0] = v.x;
      out[4 * i + 1] = v.y;
      out[4 * i + 2] = v.z;
      out[4 * i + 3] = v.w;
    }
  } else {
    if constexpr (N % 8 == 0) {
#pragma unroll
      for (int i = 0; i < N / 8; ++i) {
        uint4 v = reinterpret_cast<const uint4*>(p)[i];
        uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          out[8 * i + 2 * c + 0] = io<T>::bits_to_f32(w[c] & 0xffffu);
          out[8 * i + 2 * c + 1] = io<T>::bits_to_f32(w[c] >> 16);
        }
      }
    } else {
      static_assert(N == 4, "16-bit loads come in 4- or 8-element units");
      uint2 v = *reinterpret_cast<const uint2*>(p);
      out[0] = io<T>::bits_to_f32(v.x & 0xffffu);
      out[1] = io<T>::bits_to_f32(v.x >> 16);
      out[2] = io<T>::bits_to_f32(v.y & 0xffffu);
      out[3] = io<T>::bits_to_f32(v.y >> 16);
    }
  }
}

// bf16 specialisation of the unpack: the high half needs only a mask, the low
// half a shift (one VALU op per element instead of two).
template <>
__device__ inline void load_vec<bf16_t, 8>(const bf16_t* __restrict__ p, float (&out)[8]) {
  uint4 v = *reinterpret_cast<const uint4*>(p);
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    out[2 * c + 0] = __uint_as_float(w[c] << 16);
    out[2 * c + 1] = __uint_as_float(w[c] & 0xffff0000u);
  }
}

// Two fp32 values rounded to the 16-bit storage type and packed (lo in bits
// 0-15): one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 on gfx950, round to nearest
// even like the scalar conversions above.
template <typename T>
__device__ inline uint32_t pack2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  if constexpr (std::is_same<T, bf16_t>::value) {
    typedef __bf16 h16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, h16x2));
  } else {
    static_assert(std::is_same<T, f16_t>::value, "pack2 takes a 16-bit storage type");
    typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, h16x2));
  }
}

// STREAM: nontemporal stores, for kernels whose output is not read back soon
// (the standalone element-wise maps and the cumulative-product scan): measured
// 2-4 % faster on those read+write streams, where the read-dominated SSM lost
// time with nontemporal loads.
template <typename T, int N, bool STREAM = false>
__device__ inline void store_vec(T* __restrict__ p, const float (&in)[N]) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  if constexpr (sizeof(T) == 4) {
    static_assert(N % 4 == 0, "fp32 stores come in float4 units");
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const f32x4 v = {in[4 * i + 0], in[4 * i + 1], in[4 * i + 2], in[4 * i + 3]};
      if constexpr (STREAM)
        __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p) + i);
      else
        reinterpret_cast<f32x4*>(p)[i] = v;
    }
  } else {
    static_assert(N % 4 == 0, "16-bit stores come in 4-element units");
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const u32x2 v = {pack2<T>(in[4 * i + 0], in[4 * i + 1]), pack2<T>(in[4 * i + 2], in[4 * i + 3])};
      if constexpr (STREAM)
        __builtin_nontemporal_store(v, reinterpret_cast<u32x2*>(p) + i);
      else
        reinterpret_cast<u32x2*>(p)[i] = v;
    }
  }
}

template <typename T>
__device__ inline float load_scalar(const T* __restrict__ p) {
  return io<T>::to_f32(*p);
}

template <typename T>
__device__ inline void store_scalar(T* __restrict__ p, float v) {
  *p = io<T>::from_f32(v);
}

// ---------------------------------------------------------------------------
// Hamilton product r = p (x) q (textbook form; reference
// mambaqc/kernels/quaternion_ops.py:278-281).
// ---------------------------------------------------------------------------
struct quat { float w, x, y, z; };

__device__ inline quat qmul(const quat& p, const quat& q) {
  quat r;
  r.w = p.w * q.w - p.x * q.x - p.y * q.y - p.z * q.z;
  r.x = p.w * q.x + p.x * q.w + p.y * q.z - p.z * q.y;
  r.y = p.w * q.y - p.x * q.z + p.y * q.w + p.z * q.x;
  r.z = p.w * q.z + p.x * q.y - p.y * q.x + p.z * q.w;
  return r;
}

// acc += p (x) q
__device__ inline void qmul_acc(quat& acc, const quat& p, const quat& q) {
  acc.w = fmaf(p.w, q.w, fmaf(-p.x, q.x, fmaf(-p.y, q.y, fmaf(-p.z, q.z, acc.w))));
  acc.x = fmaf(p.w, q.x, fmaf(p.x, q.w, fmaf(p.y, q.z, fmaf(-p.z, q.y, acc.x))));
  acc.y = fmaf(p.w, q.y, fmaf(-p.x, q.z, fmaf(p.y, q.w, fmaf(p.z, q.x, acc.y))));
  acc.z = fmaf(p.w, q.z, fmaf(p.x, q.y, fmaf(-p.y, q.x, fmaf(p.z, q.w, acc.z))));
}

__device__ inline quat quat_from(const float* v) { return quat{v[0], v[1], v[2], v[3]}; }

// ---------------------------------------------------------------------------
// Cross-lane data movement on the VALU (wave64, gfx950). DPP reads a
// neighbour's register inside the consuming add (v_add_f32_dpp), and the
// permlane swaps exchange whole 16- or 32-lane rows, so none of these goes
// through the LDS pipeline the way ds_bpermute does.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ inline float dpp_mov(float v) {
  // bound_ctrl set: lets the compiler fold the move into the consumer. Every
  // pattern below reads an existing lane, so the bound control never applies.
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
// Lane i reads lane i^1 / i^2 inside its quad.
__device__ inline float lane_xor1(float v) { return dpp_mov<0xB1>(v); }  // quad_perm [1,0,3,2]
__device__ inline float lane_xor2(float v) { return dpp_mov<0x4E>(v); }  // quad_perm [2,3,0,1]
// Lane i reads lane (i - 4 or 8) mod 16 inside its 16-lane row.
__device__ inline float row_rot4(float v) { return dpp_mov<0x124>(v); }  // row_ror:4
__device__ inline float row_rot8(float v) { return dpp_mov<0x128>(v); }  // row_ror:8

// The row swaps are issued as inline assembly with both registers read-write:
// through the builtins, this compiler reads the first result in place of the
// second one when the two are added (v + v instead of v + partner). The
// s_nop pairs cover the VALU-write -> permlane-read dependency and the other
// way round.
//
// Sum over each pair of rows, delivered to the even row: lanes 0-15 receive
// v(0-15) + v(16-31) and lanes 32-47 receive v(32-47) + v(48-63); the odd
// rows receive 0.
__device__ inline float sum_row_pair_to_even(float v) {
  float a = v, b = 0.f;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  return a + b;
}
// Sum over the two 32-lane halves, delivered to lanes 0-31 (lanes 32-63 get 0).
__device__ inline float sum_halves_to_low(float v) {
  float a = v, b = 0.f;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  return a + b;
}

// ---------------------------------------------------------------------------
// XCD-aware block order. MI355X dispatches the workgroups of a launch to its 8
// XCDs (each with its own L2) round-robin by linear block id, so neighbouring
// blocks land on different L2s. Where neighbouring blocks share cache lines
// (the SSM kernels: a few d's per block, so one line of delta, s, gy, y or of
// the fp32 d_delta / d_s spans several blocks), every XCD fetches the line or
// writes part of it. This remap gives each XCD a contiguous range of logical
// blocks; it is the identity when the block count is not a multiple of 8.
// ---------------------------------------------------------------------------
constexpr int kXCDs = 8;

__device__ inline void xcd_block(int64_t& bx, int64_t& by) {
  const int64_t gx = gridDim.x;
  const int64_t n = gx * gridDim.y;
  const int64_t lin = blockIdx.x + (int64_t)blockIdx.y * gx;
  const int64_t logical = n % kXCDs ? lin : (lin % kXCDs) * (n / kXCDs) + lin / kXCDs;
  bx = logical % gx;
  by = logical / gx;
}

// ---------------------------------------------------------------------------
// Launch helpers
// ---------------------------------------------------------------------------
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? MQC_OK : (int)e;
}

inline bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Whether the byte ranges [a, a + na) and [b, b + nb) share a byte (NULL or
// empty ranges share none).
inline bool overlaps(const void* a, int64_t na, const void* b, int64_t nb) {
  if (!a || !b || na <= 0 || nb <= 0) return false;
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + (uintptr_t)nb && y < x + (uintptr_t)na;
}

// Two state buffers of n bytes that share bytes without being the same buffer:
// where a kernel allows h_last == h0 (each state written only by the lane that
// read it), a shifted alias still lets one lane overwrite another's h0 first.
inline bool partial_overlap(const void* a, const void* b, int64_t n) {
  return a != b && overlaps(a, n, b, n);
}

}  // namespace mqc
