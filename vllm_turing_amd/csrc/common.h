// Shared device helpers of the W8A8 kernels for gfx950 (CDNA4): fp16/bf16 conversions, the two scale-epilogue
// chains, int8 quantization and wavefront reductions.  Every file is compiled with -ffp-contract=off: no multiply-add
// is fused unless written as __builtin_fmaf, so each float operation below is exactly one IEEE rounding.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace w8 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

enum : int { DT_F16 = 0, DT_BF16 = 1 };

// ---- 16-bit float formats (storage is the raw bit pattern) ---------------------------------------------------------
struct f16 { uint16_t bits; };
struct bf16 { uint16_t bits; };

__device__ __forceinline__ float to_float(f16 v) {
    _Float16 h;
    __builtin_memcpy(&h, &v.bits, 2);
    return (float)h;                                   // exact
}
__device__ __forceinline__ float to_float(bf16 v) { return __uint_as_float((uint32_t)v.bits << 16); }

template <typename T> __device__ __forceinline__ uint16_t from_float(float x);
template <> __device__ __forceinline__ uint16_t from_float<f16>(float x) {
    // The barrier keeps x a rounded float32: without it the compiler folds a preceding multiply / fma and this
    // conversion into one v_fma_mixlo_f16 / v_mad_mixlo_f16, which rounds the exact result once to fp16 instead of
    // rounding to float32 first, as the reference's __float2half_rn(float) does.
    asm volatile("" : "+v"(x));
    _Float16 h = (_Float16)x;                          // v_cvt_f16_f32: IEEE round to nearest even
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}
template <> __device__ __forceinline__ uint16_t from_float<bf16>(float x) {
    // v_cvt_pk_bf16_f32 (gfx950): IEEE round to nearest even, overflow to inf, subnormals kept; one instruction
    // where the integer form takes five.  Checked on every sign / exponent / mantissa with the rounding-critical low
    // halves against torch's CPU conversion (GPU test of the f32_to_16 export).
    const __bf16 h = (__bf16)x;
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
}

__device__ __forceinline__ float lo_half(uint32_t w, f16) { return to_float(f16{(uint16_t)(w & 0xffff)}); }
__device__ __forceinline__ float hi_half(uint32_t w, f16) { return to_float(f16{(uint16_t)(w >> 16)}); }
__device__ __forceinline__ float lo_half(uint32_t w, bf16) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_half(uint32_t w, bf16) { return __uint_as_float(w & 0xffff0000u); }

// ---- scale epilogues (int32 accumulator -> float, before the final rounding to T) ----------------------------------
// Small-M chain of the GEMV / MMA kernels (csrc/w8a8_gemv.cu:91, `(float) acc * sa * sw + b` contracted by nvcc's
// default --fmad=true):  fma(RN32(float(acc) * sa), sw, b), b = +0 without a bias.
__device__ __forceinline__ float epi_small(int acc, float sa, float sw, float b) {
    const float t = (float)acc * sa;
    return __builtin_fmaf(t, sw, b);
}
// Large-M chain (csrc/w8a8_big.cu:26-35: ScaleB, then ScaleA, each rounded to float); with a bias the c2x bias
// epilogue's multiply-add of ScaleA, the ScaleB product and the bias: fma(sa, RN32(float(acc) * sw), b).
__device__ __forceinline__ float epi_large(int acc, float sa, float sw) {
    const float t = (float)acc * sw;
    return sa * t;
}
__device__ __forceinline__ float epi_large_bias(int acc, float sa, float sw, float b) {
    const float t = (float)acc * sw;
    return __builtin_fmaf(sa, t, b);
}

// ---- int8 quantization of one value: round half to even, saturate (csrc/silu_quant.cu:16-20) -----------------------
__device__ __forceinline__ int q8(float v) {
    float r = __builtin_rintf(v);                      // v_rndne_f32
    r = __builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
    return (int)r;
}
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) | ((uint32_t)d << 24);
}

// Compute units of the current device (cached per device; host threads may race on the first query, which stores
// the same value).
inline int cu_count() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cached[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// ---- buffer loads straight into LDS ----------------------------------------------------------------------------------
// s_waitcnt immediate for vmcnt(n) alone (expcnt and lgkmcnt left at their maxima; gfx9 encoding).
constexpr int waitcnt_vm(int n) { return (n & 0xf) | ((n >> 4) << 14) | 0x70 | 0xf00; }

// Raw buffer descriptor over `bytes` bytes (callers keep every offset within 31 bits).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, long bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

typedef __attribute__((address_space(3))) void lds_void;

// ---- wavefront (64-lane) reductions ----------------------------------------------------------------------------------
// DPP row operations combine lanes inside each 16-lane row, ds_swizzle combines the two rows of each 32-lane half,
// and the two halves meet through readlane.  max and integer add are exact, so the order is free.
template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_max(float v) {
    v = __builtin_fmaxf(v, dpp_f<0xB1>(v));            // quad_perm [1,0,3,2]: lane ^ 1
    v = __builtin_fmaxf(v, dpp_f<0x4E>(v));            // quad_perm [2,3,0,1]: lane ^ 2
    v = __builtin_fmaxf(v, dpp_f<0x141>(v));           // row_half_mirror: completes each group of 8
    v = __builtin_fmaxf(v, dpp_f<0x140>(v));           // row_mirror: completes each row of 16
    v = __builtin_fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)));  // lane ^ 16
    const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    return __builtin_fmaxf(lo, hi);                    // wave-uniform
}

template <int CTRL> __device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}
// Sum of an int over the 64 lanes (exact; wave-uniform result).
__device__ __forceinline__ int wave_sum(int v) {
    v += dpp_i<0xB1>(v);                               // lane ^ 1
    v += dpp_i<0x4E>(v);                               // lane ^ 2
    v += dpp_i<0x141>(v);                              // row_half_mirror: groups of 8
    v += dpp_i<0x140>(v);                              // row_mirror: rows of 16
    v += __builtin_amdgcn_ds_swizzle(v, 0x401F);       // lane ^ 16
    return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 32);
}

// ---- SiLU(gate) * up in 16 bits (silu_quant.cu:11-14,39) ------------------------------------------------------------
// silu rounded to the 16-bit type, then its exact float32 product with u (both 16-bit values) rounded once more.
__device__ __forceinline__ float silu_f(float f) {
    const float e = expf(-f);                               // HIP's float32 exp (within 2 float32 ulps here)
    const float d = 1.0f + e;
    return f / d;                                           // IEEE division
}

template <typename T>
__device__ __forceinline__ uint16_t silu_mul(float g, float u) {
    const uint16_t sh = from_float<T>(silu_f(g));
    return from_float<T>(to_float(T{sh}) * u);            // exact float product of two 16-bit values, one rounding
}

}  // namespace w8
