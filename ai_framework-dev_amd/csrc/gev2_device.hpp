// Device-side helpers shared by the gfx950 GEMM kernels: element types,
// 16-byte chunk packing, activation forward/derivative, bias loading.
//
// Activation formulas follow the reference's epilogue math
// (backends/cuda/ops/_common/shim/activations.hpp:14-70): GELU is the tanh
// form with c = 0.7978845608, k1 = 0.044715 and inner argument
// fmaf(c*k1, x^3, c*x); its derivative clamps tanh to +-0.999999; LeakyReLU'
// is `slope` at x == 0; Sigmoid is the branch-stable form.  tanh/exp are
// HIP's own device math (ocml), not a reproduction of any vendor intrinsic.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gev2 {

enum ActKind : int { kActNone = 0, kActRelu = 1, kActLeaky = 2, kActGelu = 3, kActSigmoid = 4, kActTanh = 5 };
enum BiasKind : int { kBiasNone = 0, kBiasScalar = 1, kBiasPerM = 2, kBiasPerN = 3 };
enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // one 16-byte chunk
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Raw buffer addressing and direct-to-LDS loads (buffer_load ... lds)
// ---------------------------------------------------------------------------
// Byte offset that lies outside every buffer resource made here (their range
// is 2^31 - 1 bytes): loads from it return zero, stores to it are dropped.
constexpr int kOobOffset = static_cast<int>(0x80000000u);

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Buffer resource words of a raw buffer of 2^31 - 1 bytes at `base`: an
// offset at or past 2^31 - 1 (kOobOffset) reads as zero.
__device__ __forceinline__ i32x4_t rsrc_words(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4_t r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>((a >> 32) & 0xffffu));
  r[2] = 0x7fffffff;
  r[3] = 0x00020000;
  return r;
}

// 16 bytes per lane from rsrc + voff + soff into LDS [lds_addr + 16 * lane].
// M0 is reserved to the compiler, which warns about the clobber; nothing else
// in these kernels uses M0 (LDS instructions on gfx9+ do not read it), which
// the generated code shows, so the value set here is only read by this load.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const i32x4_t& rsrc, int voff, int soff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(soff), "s"(lds_addr)
               : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

constexpr float kGeluC = 0.7978845608f;
constexpr float kGeluK1 = 0.044715f;

__device__ __forceinline__ float act_fwd(float x, int act, float slope) {
  switch (act) {
    case kActRelu: return x > 0.f ? x : 0.f;
    case kActLeaky: return x > 0.f ? x : slope * x;
    case kActGelu: {
      const float x3 = x * x * x;
      const float t = fmaf(kGeluC * kGeluK1, x3, kGeluC * x);
      return 0.5f * x * (1.f + tanhf(t));
    }
    case kActSigmoid:
      if (x >= 0.f) { const float z = expf(-x); return 1.f / (1.f + z); }
      else { const float z = expf(x); return z / (1.f + z); }
    case kActTanh: return tanhf(x);
    default: return x;
  }
}

__device__ __forceinline__ float act_grad(float x, int act, float slope) {
  switch (act) {
    case kActRelu: return x > 0.f ? 1.f : 0.f;
    case kActLeaky: return x > 0.f ? 1.f : slope;
    case kActGelu: {
      const float x2 = x * x;
      const float t = fmaf(kGeluC * kGeluK1, x2 * x, kGeluC * x);
      float th = tanhf(t);
      th = fminf(fmaxf(th, -0.999999f), 0.999999f);
      const float sech2 = 1.f - th * th;
      const float dt = kGeluC * (1.f + 3.f * kGeluK1 * x2);
      return 0.5f * (1.f + th) + 0.5f * x * sech2 * dt;
    }
    case kActSigmoid: {
      float s;
      if (x >= 0.f) { const float z = expf(-x); s = 1.f / (1.f + z); }
      else { const float z = expf(x); s = z / (1.f + z); }
      return s * (1.f - s);
    }
    case kActTanh: { const float th = tanhf(x); return 1.f - th * th; }
    default: return 1.f;
  }
}

// ---------------------------------------------------------------------------
// Element traits.  A "chunk" is 16 bytes: 8 half-precision or 4 fp32 values.
// ---------------------------------------------------------------------------
template <typename T> struct Elem;

template <> struct Elem<float> {
  static constexpr int kPerChunk = 4;
  __device__ __forceinline__ static float load1(const void* p) { return *reinterpret_cast<const float*>(p); }
  __device__ __forceinline__ static uint32_t bits(float v) { return __float_as_uint(v); }
  __device__ __forceinline__ static void store1(void* p, float v) { *reinterpret_cast<float*>(p) = v; }
};

template <> struct Elem<__bf16> {
  static constexpr int kPerChunk = 8;
  __device__ __forceinline__ static float from_bits(uint32_t h) { return __uint_as_float(h << 16); }
  __device__ __forceinline__ static uint32_t bits(float v) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(v)));
  }
  __device__ __forceinline__ static float load1(const void* p) {
    return from_bits(*reinterpret_cast<const uint16_t*>(p));
  }
  __device__ __forceinline__ static void store1(void* p, float v) {
    *reinterpret_cast<uint16_t*>(p) = static_cast<uint16_t>(bits(v));
  }
};

template <> struct Elem<_Float16> {
  static constexpr int kPerChunk = 8;
  __device__ __forceinline__ static float from_bits(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
  }
  __device__ __forceinline__ static uint32_t bits(float v) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(v)));
  }
  __device__ __forceinline__ static float load1(const void* p) {
    return from_bits(*reinterpret_cast<const uint16_t*>(p));
  }
  __device__ __forceinline__ static void store1(void* p, float v) {
    *reinterpret_cast<uint16_t*>(p) = static_cast<uint16_t>(bits(v));
  }
};

// Unpack a chunk into fp32 values.
template <typename T>
__device__ __forceinline__ void chunk_to_f32(const u32x4& c, float* v) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(c[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t w = c[i];
      v[2 * i] = Elem<T>::from_bits(w & 0xffffu);
      v[2 * i + 1] = Elem<T>::from_bits(w >> 16);
    }
  }
}

// Pack fp32 values (rounded once, RNE) into a chunk.
template <typename T>
__device__ __forceinline__ u32x4 f32_to_chunk(const float* v) {
  u32x4 c;
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = __float_as_uint(v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      c[i] = Elem<T>::bits(v[2 * i]) | (Elem<T>::bits(v[2 * i + 1]) << 16);
  }
  return c;
}

// Compile-time activation forms (same formulas as act_fwd / act_grad) so that
// loops over register tiles unroll fully; dispatch_act() picks one at run time.
template <int ACT>
__device__ __forceinline__ float act_fwd_t(float x, float slope) { return act_fwd(x, ACT, slope); }
template <int ACT>
__device__ __forceinline__ float act_grad_t(float x, float slope) { return act_grad(x, ACT, slope); }

template <typename F>
__device__ __forceinline__ void dispatch_act(int act, F&& f) {
  switch (act) {
    case kActRelu: f.template operator()<kActRelu>(); break;
    case kActLeaky: f.template operator()<kActLeaky>(); break;
    case kActGelu: f.template operator()<kActGelu>(); break;
    case kActSigmoid: f.template operator()<kActSigmoid>(); break;
    case kActTanh: f.template operator()<kActTanh>(); break;
    default: f.template operator()<kActNone>(); break;
  }
}

// Run-time choice among the piecewise-linear activations only (none, ReLU,
// LeakyReLU); any other kind is treated as none.
template <typename F>
__device__ __forceinline__ void dispatch_act_linear(int act, F&& f) {
  switch (act) {
    case kActRelu: f.template operator()<kActRelu>(); break;
    case kActLeaky: f.template operator()<kActLeaky>(); break;
    default: f.template operator()<kActNone>(); break;
  }
}

__device__ __forceinline__ float load_bias(const float* bias, int kind, int m, int n) {
  switch (kind) {
    case kBiasScalar: return bias[0];
    case kBiasPerM: return bias[m];
    case kBiasPerN: return bias[n];
    default: return 0.f;
  }
}

}  // namespace gev2
