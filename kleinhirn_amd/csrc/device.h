// Device helpers shared by the kernels: storage loads/stores with f32 arithmetic, wavefront
// reductions (64 lanes on CDNA4) and the activation functions of the plan's matmul ACT codes.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace kh {

typedef _Float16 half_t;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int WAVE = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// v of lane ^ 32 (the other half of the wavefront). The lane id is read where the exchange runs
// (a volatile asm the compiler does not hoist), so no index register stays live across the
// caller's loops, and ds_bpermute needs no bounds handling for an in-wave partner.
__device__ __forceinline__ float xor32(float v) {
  int lane;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane));
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __float_as_int(v)));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Work item of block b in a 1-D grid of nblk blocks: the dispatcher sends block b to XCD b % 8, so
// each XCD gets a contiguous range of items (neighbouring items share operands in that XCD's L2).
__device__ __forceinline__ int xcd_tile(int tile, int nblk) {
  const int per = (nblk + 7) / 8;
  const int x = tile % 8, i = tile / 8;
  const int full = nblk - (per - 1) * 8;  // XCDs that hold `per` items (the rest hold per - 1)
  return x < full ? x * per + i : full * per + (x - full) * (per - 1) + i;
}

// GELU by erf through Abramowitz-Stegun 7.1.26 (the reference's constants, src/wasm/plan.ts:99-107)
// erf(x) = 1 - P(t) exp(-x^2), t = 1 / (1 + p x) for x = |v| / sqrt 2 >= 0, so with
// R = P exp(-v^2 / 2) / 2: gelu(v) = v - v R for v >= 0 and v R below. The 1/2 is folded into the
// polynomial's coefficients (exact: a power of two), 1/sqrt 2 into p and the exponent goes to the
// hardware exp2; 12 VALU operations and two transcendentals per value, within 5e-7 of the
// reference's arrangement of the same formula.
__device__ __forceinline__ float gelu_as(float v) {
  // hardware reciprocal (1 ulp): the formula's own error is 1.5e-7 absolute
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f * 0.7071067811865476f, fabsf(v), 1.0f));
  float p = __builtin_fmaf(0.5f * 1.061405429f, t, 0.5f * -1.453152027f);
  p = __builtin_fmaf(p, t, 0.5f * 1.421413741f);
  p = __builtin_fmaf(p, t, 0.5f * -0.284496736f);
  p = __builtin_fmaf(p, t, 0.5f * 0.254829592f);
  p = p * t;
  const float e = __builtin_amdgcn_exp2f((v * v) * (-0.5f * 1.4426950408889634f));
  // w carries the sign of v: max(v, 0) - |w| is v - w for v >= 0 and w below
  const float w = v * (p * e);
  return fmaxf(v, 0.0f) - fabsf(w);
}

__device__ __forceinline__ float activate(float v, int act) {
  switch (act) {
    case 1: return fmaxf(v, 0.0f);
    case 2: return gelu_as(v);
    case 3: return tanhf(v);
    case 4: return v / (1.0f + __expf(-v));
    default: return v;
  }
}

template <typename T>
__device__ __forceinline__ float ldf(const T *p, int64_t i) { return (float)p[i]; }
template <typename T>
__device__ __forceinline__ void stf(T *p, int64_t i, float v) { p[i] = (T)v; }

// VEC contiguous storage elements as f32
template <typename T, int VEC>
struct VecIO;

template <>
struct VecIO<half_t, 4> {
  __device__ static void load(const half_t *p, float *o) {
    half4v v = *reinterpret_cast<const half4v *>(p);
    o[0] = (float)v[0]; o[1] = (float)v[1]; o[2] = (float)v[2]; o[3] = (float)v[3];
  }
  __device__ static void store(half_t *p, const float *o) {
    half4v v;
    v[0] = (half_t)o[0]; v[1] = (half_t)o[1]; v[2] = (half_t)o[2]; v[3] = (half_t)o[3];
    *reinterpret_cast<half4v *>(p) = v;
  }
};
template <>
struct VecIO<half_t, 2> {
  __device__ static void load(const half_t *p, float *o) {
    half2v v = *reinterpret_cast<const half2v *>(p);
    o[0] = (float)v[0]; o[1] = (float)v[1];
  }
  __device__ static void store(half_t *p, const float *o) {
    half2v v;
    v[0] = (half_t)o[0]; v[1] = (half_t)o[1];
    *reinterpret_cast<half2v *>(p) = v;
  }
};
template <>
struct VecIO<half_t, 8> {
  __device__ static void load(const half_t *p, float *o) {
    half8v v = *reinterpret_cast<const half8v *>(p);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = (float)v[i];
  }
  __device__ static void store(half_t *p, const float *o) {
    half8v v;
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (half_t)o[i];
    *reinterpret_cast<half8v *>(p) = v;
  }
};
template <>
struct VecIO<float, 4> {
  __device__ static void load(const float *p, float *o) {
    float4v v = *reinterpret_cast<const float4v *>(p);
    o[0] = v[0]; o[1] = v[1]; o[2] = v[2]; o[3] = v[3];
  }
  __device__ static void store(float *p, const float *o) {
    float4v v;
    v[0] = o[0]; v[1] = o[1]; v[2] = o[2]; v[3] = o[3];
    *reinterpret_cast<float4v *>(p) = v;
  }
};
template <>
struct VecIO<float, 2> {
  __device__ static void load(const float *p, float *o) {
    float2v v = *reinterpret_cast<const float2v *>(p);
    o[0] = v[0]; o[1] = v[1];
  }
  __device__ static void store(float *p, const float *o) {
    float2v v;
    v[0] = o[0]; v[1] = o[1];
    *reinterpret_cast<float2v *>(p) = v;
  }
};
template <typename T>
struct VecIO<T, 1> {
  __device__ static void load(const T *p, float *o) { o[0] = (float)p[0]; }
  __device__ static void store(T *p, const float *o) { p[0] = (T)o[0]; }
};

}  // namespace kh
