// AR8: the compressed operand of the reference's large all-reduce (csrc/host_ar.cu:133-201), int8 with an fp16 scale
// per 128-element group, about half the bytes of fp16 on the wire.  Each rank quantizes its operand, the packed blocks
// are all-gathered (the collective itself is not part of this library), and every rank sums the dequantised blocks
// of all ranks in rank order, so the result is identical everywhere.
//
// Arithmetic (bit-exact contract), per 128-element group g of an fp16 vector x (n % 128 == 0):
//   amax = max |float(x)|, scale = RN16(amax / 127), s = float(scale), inv = s > 0 ? 1 / s : 0 (IEEE division),
//   q = clamp(rint(float(x) * inv), -127, 127);  packed = [q: n int8][scale: n / 128 fp16]
//   out = RN16(sum over ranks r of q_r * s_r): the products are exact in float32 (8-bit by 11-bit significands); the
//   float32 sum runs in rank order as fused multiply-adds, which for the reference's two ranks is its single rounding
//   of u * a0 + w * a1.
//
// HBM-bound byte work.  Quantization: 16 lanes (one DPP row) per group, 8 elements per lane in one 16-byte load; the
// group's absmax is reduced with four DPP row operations, so a wavefront quantizes 4 groups with no LDS and no
// barrier.  Dequantisation: 8 elements per lane, one 8-byte load per rank plus the group's scale.
#include "common.h"
#include "../../include/w8a8_mi355.h"

namespace w8 {

constexpr int AR8_GROUP = 128;
constexpr int AR8_MAX_RANKS = 8;

__device__ __forceinline__ float row16_max(float v) {
    v = __builtin_fmaxf(v, dpp_f<0xB1>(v));            // lane ^ 1
    v = __builtin_fmaxf(v, dpp_f<0x4E>(v));            // lane ^ 2
    v = __builtin_fmaxf(v, dpp_f<0x141>(v));           // row_half_mirror: groups of 8
    v = __builtin_fmaxf(v, dpp_f<0x140>(v));           // row_mirror: the 16-lane row
    return v;
}

__global__ void __launch_bounds__(256) ar8_quant_kernel(const uint16_t* __restrict__ x, int8_t* __restrict__ q,
                                                        uint16_t* __restrict__ scales, long ngroups) {
    const long t = blockIdx.x * (long)blockDim.x + threadIdx.x;
    const long g = t >> 4;                              // 16 lanes per group
    const int l = threadIdx.x & 15;
    const bool live = g < ngroups;                      // whole 16-lane rows are live or not together
    const uint4 v = live ? reinterpret_cast<const uint4*>(x)[g * 16 + l] : make_uint4(0, 0, 0, 0);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float f[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        f[2 * e] = lo_half(w[e], f16{});
        f[2 * e + 1] = hi_half(w[e], f16{});
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(f[i]));
    amax = row16_max(amax);
    const uint16_t sh = from_float<f16>(amax / 127.0f);
    const float s = to_float(f16{sh});
    const float inv = s > 0.0f ? 1.0f / s : 0.0f;
    int b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float r = __builtin_rintf(f[i] * inv);
        r = __builtin_fminf(__builtin_fmaxf(r, -127.0f), 127.0f);
        b[i] = (int)r;
    }
    if (live) {
        reinterpret_cast<uint2*>(q)[g * 16 + l] = make_uint2(pack4(b[0], b[1], b[2], b[3]), pack4(b[4], b[5], b[6], b[7]));
        if (l == 0) scales[g] = sh;
    }
}

template <int R>
__global__ void __launch_bounds__(256) ar8_dequant_sum_kernel(const int8_t* __restrict__ gathered,
                                                              uint16_t* __restrict__ out, long n) {
    const long t = blockIdx.x * (long)blockDim.x + threadIdx.x;   // 8 elements per thread
    if (t * 8 >= n) return;
    const long m = n + n / 64;                                    // bytes per rank block
    const long g = (t * 8) / AR8_GROUP;
    float acc[8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int8_t* base = gathered + r * m;
        const uint2 qv = reinterpret_cast<const uint2*>(base)[t];
        const float s = to_float(f16{reinterpret_cast<const uint16_t*>(base + n)[g]});
        const uint32_t w[2] = {qv.x, qv.y};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float qf = (float)(int8_t)((w[i >> 2] >> (8 * (i & 3))) & 0xff);
            acc[i] = r == 0 ? qf * s : __builtin_fmaf(qf, s, acc[i]);   // exact product; rank-order sum
        }
    }
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (uint32_t)from_float<f16>(acc[2 * e]) | ((uint32_t)from_float<f16>(acc[2 * e + 1]) << 16);
    reinterpret_cast<uint4*>(out)[t] = make_uint4(o[0], o[1], o[2], o[3]);
}

static int ar8_sum(const void* gathered, void* out, long n, int ranks, hipStream_t st) {
    const long threads = n / 8;
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    const int8_t* gp = static_cast<const int8_t*>(gathered);
    uint16_t* op = static_cast<uint16_t*>(out);
    switch (ranks) {
#define W8_CASE(R) case R: ar8_dequant_sum_kernel<R><<<blocks, 256, 0, st>>>(gp, op, n); break;
        W8_CASE(1) W8_CASE(2) W8_CASE(3) W8_CASE(4) W8_CASE(5) W8_CASE(6) W8_CASE(7) W8_CASE(8)
#undef W8_CASE
        default: return -1;
    }
    return (int)hipGetLastError();
}

}  // namespace w8

using namespace w8;

// AR8 group quantization (csrc/host_ar.cu:186-192: same arguments).  x: n fp16, packed: n int8 then n / 128 fp16
// scales (n + n / 64 bytes).  n % 128 == 0, x 16-byte and packed 8-byte aligned.  Returns 0, -1 on bad arguments,
// else the HIP launch error.
extern "C" int ar8_quant(const void* x, void* packed, int n, void* stream) {
    if (n < 0 || n % AR8_GROUP != 0 || !x || !packed || (uintptr_t)x % 16 != 0 || (uintptr_t)packed % 8 != 0) return -1;
    if (n == 0) return 0;
    const long ngroups = n / AR8_GROUP;
    const unsigned blocks = (unsigned)((ngroups * 16 + 255) / 256);
    ar8_quant_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(static_cast<const uint16_t*>(x),
                                                              static_cast<int8_t*>(packed),
                                                              reinterpret_cast<uint16_t*>(static_cast<int8_t*>(packed) + n),
                                                              ngroups);
    return (int)hipGetLastError();
}

// The sum of two ranks' dequantised blocks (csrc/host_ar.cu:194-201: same arguments).  gathered: two packed blocks in
// rank order, n + n / 64 bytes each; out: n fp16.
extern "C" int ar8_dequant_sum(const void* gathered, void* out, int n, void* stream) {
    return ar8_dequant_sum_ranks(gathered, out, n, 2, stream);
}

// The same for 1..8 ranks (no counterpart in the reference, which is two-rank only).
extern "C" int ar8_dequant_sum_ranks(const void* gathered, void* out, int n, int ranks, void* stream) {
    if (n < 0 || n % AR8_GROUP != 0 || ranks < 1 || ranks > AR8_MAX_RANKS || !gathered || !out ||
        (uintptr_t)gathered % 8 != 0 || (uintptr_t)out % 16 != 0)
        return -1;
    if (n == 0) return 0;
    return ar8_sum(gathered, out, n, ranks, (hipStream_t)stream);
}
