// ipc_device.h - device helpers shared by the iPC kernels (gfx950 only).
//
// Element types, conversions, the fused activations of
// src/ipc_tilelang/tilelang_kernels.py:61-96 (activations.py:9-29) evaluated
// in fp32, and thin wrappers over the CDNA4 MFMA builtins.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ipc {

typedef _Float16 f16;
typedef __bf16 bf16;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

enum { ACT_IDENTITY = 0, ACT_RELU = 1, ACT_TANH = 2, ACT_SIGMOID = 3, ACT_SILU = 4, ACT_GELU = 5 };

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(f16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(bf16 v) { return (float)v; }

// Rounds the fp32 value v to the operand type.  v is pinned in a register
// first: otherwise the compiler may fold the multiply that produced v into the
// conversion (v_fma_mix*, one rounding of the exact product), and the same
// source would then round differently in different kernels.
template <typename T> __device__ __forceinline__ T cvt(float v);
template <> __device__ __forceinline__ float cvt<float>(float v) { return v; }
template <> __device__ __forceinline__ f16 cvt<f16>(float v) {
  asm("" : "+v"(v));
  return (f16)v;
}
template <> __device__ __forceinline__ bf16 cvt<bf16>(float v) {
  asm("" : "+v"(v));
  return (bf16)v;
}

// Loads 4 consecutive elements (aligned to 4 elements) and widens them to fp32.
__device__ __forceinline__ void load4(const float* p, float o[4]) {
  const float4 v = *reinterpret_cast<const float4*>(p);
  o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
}
__device__ __forceinline__ float h2f(uint32_t bits16, f16*) {
  return (float)__builtin_bit_cast(f16, (uint16_t)bits16);
}
__device__ __forceinline__ float h2f(uint32_t bits16, bf16*) {
  return __builtin_bit_cast(float, bits16 << 16);
}
template <typename T>
__device__ __forceinline__ void load4_16(const T* p, float o[4]) {
  const uint2 v = *reinterpret_cast<const uint2*>(p);
  o[0] = h2f(v.x & 0xffffu, (T*)nullptr);
  o[1] = h2f(v.x >> 16, (T*)nullptr);
  o[2] = h2f(v.y & 0xffffu, (T*)nullptr);
  o[3] = h2f(v.y >> 16, (T*)nullptr);
}
__device__ __forceinline__ void load4(const f16* p, float o[4]) { load4_16(p, o); }
__device__ __forceinline__ void load4(const bf16* p, float o[4]) { load4_16(p, o); }

// ---------------------------------------------------------------- activations
// fp32 evaluation as in tilelang_kernels.py:61-96.  exp is the HIP device
// library's expf; tanh is tanh_f32 below.  Contraction into FMA is off in
// every activation, so that a function gives the same bits in every kernel it
// is inlined into (the whole-step kernels keep copies of one state in several
// workgroups and must agree on them exactly).

// tanh in fp32, branch-free: for |x| < 0.55, x + x^3 P(x^2) with P of degree 4
// fitted to tanh(a)/a - 1 on [0, 0.55] (relative approximation error 1e-9);
// above, 1 - 2 / (exp(2|x|) + 1) with the hardware exp2 and reciprocal, which
// lose at most ~2 ulp to the cancellation just above 0.55; the sign is
// restored at the end.  Within 2 ulp of tanh over float32 in a CPU model of
// the operations (100 M points against float64 tanh, correctly rounded exp2
// and reciprocal); tanh(+-inf) = +-1, NaN stays NaN.  About half the
// instructions of the device library's two-branch tanhf, whose lanes diverge.
__device__ __forceinline__ float tanh_f32(float x) {
#pragma clang fp contract(off)
  const float a = __builtin_fabsf(x), s = a * a;
  float p = __builtin_fmaf(-0.00628247811f, s, 0.0210777614f);
  p = __builtin_fmaf(p, s, -0.0538538583f);
  p = __builtin_fmaf(p, s, 0.133326024f);
  p = __builtin_fmaf(p, s, -0.333333194f);
  const float small = __builtin_fmaf(a, s * p, a);
  const float e = __builtin_amdgcn_exp2f(a * 2.88539004f);  // exp(2a)
  const float large = __builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
  return __builtin_copysignf(a < 0.55f ? small : large, x);
}

__device__ __forceinline__ float sigmoidf_(float x) {
#pragma clang fp contract(off)
  return 1.0f / (1.0f + expf(-x));
}

__device__ __forceinline__ float act_f(int act, float x) {
#pragma clang fp contract(off)
  switch (act) {
    case ACT_RELU: return x > 0.0f ? x : 0.0f;
    case ACT_TANH: return tanh_f32(x);
    case ACT_SIGMOID: return sigmoidf_(x);
    case ACT_SILU: return x * sigmoidf_(x);
    case ACT_GELU: {
      const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
      return 0.5f * x * (1.0f + tanh_f32(u));
    }
    default: return x;
  }
}

__device__ __forceinline__ float act_df(int act, float x) {
#pragma clang fp contract(off)
  switch (act) {
    case ACT_RELU: return x > 0.0f ? 1.0f : 0.0f;
    case ACT_TANH: { const float y = tanh_f32(x); return 1.0f - y * y; }
    case ACT_SIGMOID: { const float y = sigmoidf_(x); return y * (1.0f - y); }
    case ACT_SILU: { const float s = sigmoidf_(x); return s * (1.0f + x * (1.0f - s)); }
    case ACT_GELU: {
      const float c = 0.044715f, k = 0.7978845608028654f;
      const float u = k * (x + c * x * x * x);
      const float t = tanh_f32(u);
      const float du = k * (1.0f + 3.0f * c * x * x);
      return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * du;
    }
    default: return 1.0f;
  }
}

// Compile-time forms of the same activations, for kernels instantiated per
// activation (no switch in their inner loops).
template <int ACT> __device__ __forceinline__ float act_t(float x) {
#pragma clang fp contract(off)
  if (ACT == ACT_RELU) return x > 0.0f ? x : 0.0f;
  if (ACT == ACT_TANH) return tanh_f32(x);
  if (ACT == ACT_SIGMOID) return sigmoidf_(x);
  if (ACT == ACT_SILU) return x * sigmoidf_(x);
  if (ACT == ACT_GELU) {
    const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    return 0.5f * x * (1.0f + tanh_f32(u));
  }
  return x;
}

template <int ACT> __device__ __forceinline__ float dact_t(float x) {
#pragma clang fp contract(off)
  if (ACT == ACT_RELU) return x > 0.0f ? 1.0f : 0.0f;
  if (ACT == ACT_TANH) { const float y = tanh_f32(x); return 1.0f - y * y; }
  if (ACT == ACT_SIGMOID) { const float y = sigmoidf_(x); return y * (1.0f - y); }
  if (ACT == ACT_SILU) { const float s = sigmoidf_(x); return s * (1.0f + x * (1.0f - s)); }
  if (ACT == ACT_GELU) {
    const float c = 0.044715f, k = 0.7978845608028654f;
    const float u = k * (x + c * x * x * x);
    const float t = tanh_f32(u);
    const float du = k * (1.0f + 3.0f * c * x * x);
    return 0.5f * (1.0f + t) + 0.5f * x * (1.0f - t * t) * du;
  }
  return 1.0f;
}

// f'(x) given y = act_t<ACT>(x) already evaluated: the same bits as
// dact_t<ACT>(x) (tanh and sigmoid reuse y, the others evaluate f'(x) anew).
template <int ACT> __device__ __forceinline__ float dact_from_t(float x, float y) {
#pragma clang fp contract(off)
  if (ACT == ACT_TANH) return 1.0f - y * y;
  if (ACT == ACT_SIGMOID) return y * (1.0f - y);
  return dact_t<ACT>(x);
}

// ---------------------------------------------------------------- MFMA
// 32x32 output block per wave.  Operand lane layout (both operands): lane l
// supplies row/column (l % 32) and the k-slice (l / 32) of the instruction's
// K; the fp32 result element j of lane l is C[8*(j/4) + 4*(l/32) + j%4][l%32].
template <typename OT> struct Mfma32;

template <> struct Mfma32<float> {
  static constexpr int KI = 2;    // k per instruction
  static constexpr int KPL = 1;   // k values per lane
  typedef float operand;
  __device__ __forceinline__ static f32x16 run(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma32<f16> {
  static constexpr int KI = 16;
  static constexpr int KPL = 8;
  typedef f16x8 operand;
  __device__ __forceinline__ static f32x16 run(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma32<bf16> {
  static constexpr int KI = 16;
  static constexpr int KPL = 8;
  typedef bf16x8 operand;
  __device__ __forceinline__ static f32x16 run(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

}  // namespace ipc
