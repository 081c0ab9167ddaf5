// Per-token dynamic int8 quantization of W8A8 activations, and the fused SiLU(gate) * up + quantization of the MLP
// down projection's input, for gfx950.
//
// Both are single-pass row reductions: the row is read once from HBM with 16-byte loads into registers, its absmax
// is reduced inside the wavefront with DPP / ds_swizzle (and across the wavefronts of a block through LDS), and the
// int8 row is written from the same registers.  HBM traffic is the algorithmic minimum: 2 bytes in and 1 byte out per
// element (3 in for the SiLU kernel) plus a float32 scale per row.
//
// Arithmetic (bit-exact contract):
//   absmax = max |float(x)|, inverse = absmax > 0 ? 127 / absmax : 0 (IEEE division), scale = absmax / 127,
//   q = clamp(rint(float(x) * inverse), -128, 127)
// following vllm_turing/quantfuse.py:18-24 and csrc/silu_quant.cu:57-58,66 (zero-row rule).  The SiLU kernel computes
// r = RN_T(float(silu(g)) * float(u)) with silu(g) = RN_T(f / (1 + expf(-f))) as csrc/silu_quant.cu:11-14,39 does.
// silu depends only on the 16-bit input, so it is checked exhaustively: on all 65,536 fp16 and all 65,536 bf16 inputs
// the float32 result of this expression is within 2 float32 ulps of the one built on a correctly rounded exp and
// rounds to the same 16-bit value (GPU test against the oracle's table).  For the same reason the SiLU kernel that
// normally runs looks silu up in a table of all 65,536 16-bit results per type, generated at build time from the
// correctly rounded definition (vllm_turing_amd/silu_table.py into silu_table.inc), compiled in as read-only device
// data and held in LDS: the same 16-bit values as evaluating it, at a third of the VALU work, with no set-up.
//
// A third kernel fuses the residual add and the RMSNorm in front of the quantization (vLLM's
// rms_norm_dynamic_per_token_quant as vllm_turing/tailoverlap.py:145 calls it): s = x + r (float), r <- RN_T(s),
// rms = 1 / sqrt(RN32(sum s^2 / K) + eps) with the sum of squares in float64 (each square exact, the sum order-free to
// ~1e-12), y = RN_T(float(RN_T(s * rms)) * w), scale = max(absmax(y) / 127, FLT_EPSILON), q = rint(y * (1 / scale)).
#include <float.h>

#include <type_traits>

#include "common.h"
#include "../../include/w8a8_mi355.h"

namespace w8 {

constexpr int MAX_VPT_QUANT = 16;   // 16-byte vectors per thread kept in registers
constexpr int MAX_VPT_SILU = 8;

__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int nw = blockDim.x >> 6;
    if (nw == 1) return v;
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
    for (int i = 1; i < nw; ++i) m = __builtin_fmaxf(m, red[i]);
    return m;
}

// ---- per-token quant: one block per row, the row in registers ------------------------------------------------------
template <typename T, int VPT>
__global__ void __launch_bounds__(1024) per_token_quant_kernel(const uint16_t* __restrict__ x, int8_t* __restrict__ q,
                                                               float* __restrict__ scales, int K, long ldx) {
    __shared__ float red[16];
    const long row = blockIdx.x;
    const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
    const int nvec = K >> 3;
    uint4 v[VPT];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int idx = threadIdx.x + j * blockDim.x;
        v[j] = idx < nvec ? xr[idx] : make_uint4(0, 0, 0, 0);
        const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            amax = __builtin_fmaxf(amax, __builtin_fabsf(lo_half(w[e], T{})));
            amax = __builtin_fmaxf(amax, __builtin_fabsf(hi_half(w[e], T{})));
        }
    }
    amax = block_max(amax, red);
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    if (threadIdx.x == 0) scales[row] = amax / 127.0f;
    uint2* qo = reinterpret_cast<uint2*>(q + row * (long)K);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int idx = threadIdx.x + j * blockDim.x;
        if (idx < nvec) {
            const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
            int b[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                b[2 * e] = q8(lo_half(w[e], T{}) * inv);
                b[2 * e + 1] = q8(hi_half(w[e], T{}) * inv);
            }
            qo[idx] = make_uint2(pack4(b[0], b[1], b[2], b[3]), pack4(b[4], b[5], b[6], b[7]));
        }
    }
}

// Any K and alignment: element loop, the row read twice (second read from L2).
template <typename T>
__global__ void __launch_bounds__(256) per_token_quant_any_kernel(const uint16_t* __restrict__ x, int8_t* __restrict__ q,
                                                                  float* __restrict__ scales, int K, long ldx) {
    __shared__ float red[16];
    const long row = blockIdx.x;
    const uint16_t* xr = x + row * ldx;
    float amax = 0.0f;
    for (int k = threadIdx.x; k < K; k += blockDim.x) amax = __builtin_fmaxf(amax, __builtin_fabsf(to_float(T{xr[k]})));
    amax = block_max(amax, red);
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    if (threadIdx.x == 0) scales[row] = amax / 127.0f;
    for (int k = threadIdx.x; k < K; k += blockDim.x) q[row * (long)K + k] = (int8_t)q8(to_float(T{xr[k]}) * inv);
}

// ---- SiLU(gate) * up + per-token quant (silu_f, silu_mul: common.h) -------------------------------------------------

template <typename T, int VPT>
__global__ void __launch_bounds__(1024) silu_mul_quant_kernel(const uint16_t* __restrict__ gu, int8_t* __restrict__ q,
                                                              float* __restrict__ scales, int I) {
    __shared__ float red[16];
    const long row = blockIdx.x;
    const uint4* g4 = reinterpret_cast<const uint4*>(gu + row * 2 * (long)I);
    const uint4* u4 = reinterpret_cast<const uint4*>(gu + row * 2 * (long)I + I);
    const int nvec = I >> 3;
    // every vector of the row loaded first, unconditionally (past the row's end: the last vector, unused); loaded
    // under the idx < nvec branch, each was waited for before the next was issued
    uint4 gvs[VPT], uvs[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int idx = min((int)threadIdx.x + j * (int)blockDim.x, nvec - 1);
        gvs[j] = g4[idx];
        uvs[j] = u4[idx];
    }
    uint4 r[VPT];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int idx = threadIdx.x + j * blockDim.x;
        uint32_t o[4] = {0, 0, 0, 0};
        if (idx < nvec) {
            const uint4 gv = gvs[j], uv = uvs[j];
            const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
            const uint32_t uw[4] = {uv.x, uv.y, uv.z, uv.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint16_t lo = silu_mul<T>(lo_half(gw[e], T{}), lo_half(uw[e], T{}));
                const uint16_t hi = silu_mul<T>(hi_half(gw[e], T{}), hi_half(uw[e], T{}));
                o[e] = (uint32_t)lo | ((uint32_t)hi << 16);
                amax = __builtin_fmaxf(amax, __builtin_fabsf(lo_half(o[e], T{})));
                amax = __builtin_fmaxf(amax, __builtin_fabsf(hi_half(o[e], T{})));
            }
        }
        r[j] = make_uint4(o[0], o[1], o[2], o[3]);
    }
    amax = block_max(amax, red);
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    if (threadIdx.x == 0) scales[row] = amax / 127.0f;
    uint2* qo = reinterpret_cast<uint2*>(q + row * (long)I);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int idx = threadIdx.x + j * blockDim.x;
        if (idx < nvec) {
            const uint32_t w[4] = {r[j].x, r[j].y, r[j].z, r[j].w};
            int b[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                b[2 * e] = q8(lo_half(w[e], T{}) * inv);
                b[2 * e + 1] = q8(hi_half(w[e], T{}) * inv);
            }
            qo[idx] = make_uint2(pack4(b[0], b[1], b[2], b[3]), pack4(b[4], b[5], b[6], b[7]));
        }
    }
}

// ---- SiLU * up + quant through a table of the 16-bit silu --------------------------------------------------------
// silu is rounded to 16 bits before the product, so it is a function of the 16-bit gate pattern alone: its value for
// all 65,536 patterns of each type is generated at build time (silu_table.inc, fp16 first, then bf16), and a
// persistent block per CU copies the 128 KB table of its dtype into LDS and looks the gate up.  ~12 VALU instructions
// per element instead of ~42, which takes the kernel from VALU-bound to HBM-bound at prefill sizes.
constexpr int LUT_ENTRIES = 65536;
__device__ __align__(16) const uint16_t g_silu_lut[2][LUT_ENTRIES] = {
#include "silu_table.inc"
};

// silu of every 16-bit input pattern (test export): dtype 0 / 1 the device's own arithmetic (the exhaustive check of
// silu_f), 2 / 3 a copy of the compiled-in table of dtype 0 / 1.
template <typename T>
__global__ void silu_table_kernel(uint16_t* __restrict__ out, int table) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < LUT_ENTRIES)
        out[i] = table ? g_silu_lut[std::is_same<T, bf16>::value ? DT_BF16 : DT_F16][i]
                       : from_float<T>(silu_f(to_float(T{(uint16_t)i})));
}

// The table of dtype dt into LDS by direct-to-LDS loads: 128 loads of 1 KB shared out over the block's wavefronts,
// all in flight at once (a plain device function: in a template the buffer-descriptor type drops the host stub).
__device__ __forceinline__ void silu_lut_fill(uint8_t* lds, int dt) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(g_silu_lut[dt], LUT_ENTRIES * 2);
    const int lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    for (int blk = threadIdx.x >> 6; blk < LUT_ENTRIES * 2 / 1024; blk += nw)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(lds + blk * 1024), 16, blk * 1024 + lane * 16, 0, 0, 0);
}
constexpr int LUT_LDS_BYTES = LUT_ENTRIES * 2 + 2 * 16 * 4;   // the table, then two reduction buffers

template <typename T>
__device__ __forceinline__ uint32_t silu_mul_lut2(const uint16_t* lut, uint32_t g2, uint32_t u2, float& amax) {
    const uint16_t lo = from_float<T>(to_float(T{lut[g2 & 0xffff]}) * lo_half(u2, T{}));
    const uint16_t hi = from_float<T>(to_float(T{lut[g2 >> 16]}) * hi_half(u2, T{}));
    const uint32_t o = (uint32_t)lo | ((uint32_t)hi << 16);
    amax = __builtin_fmaxf(amax, __builtin_fabsf(lo_half(o, T{})));
    amax = __builtin_fmaxf(amax, __builtin_fabsf(hi_half(o, T{})));
    return o;
}

// Block b takes rows b, b + gridDim.x, ...; the next row's gate and up vectors are loaded (into the other register
// buffer) before the current row is computed, so the loads overlap its table lookups, reduction and stores.
template <typename T, int VPT>
__global__ void __launch_bounds__(1024) silu_mul_quant_lut_kernel(const uint16_t* __restrict__ gu,
                                                                  int8_t* __restrict__ q, float* __restrict__ scales,
                                                                  int M, int I) {
    extern __shared__ uint4 lds_lut[];
    uint16_t* lut = reinterpret_cast<uint16_t*>(lds_lut);
    float* red = reinterpret_cast<float*>(lut + LUT_ENTRIES);
    silu_lut_fill(reinterpret_cast<uint8_t*>(lds_lut), std::is_same<T, bf16>::value ? DT_BF16 : DT_F16);

    const int nvec = I >> 3;
    uint4 gv[2][VPT], uv[2][VPT];
    // unconditional loads (a vector past the row's end reads the last one and is not used): a load under a branch
    // makes the compiler wait for every outstanding load there, the next row's prefetch included
    auto load = [&](int b, long row) {
        const uint4* g4 = reinterpret_cast<const uint4*>(gu + row * 2 * (long)I);
        const uint4* u4 = reinterpret_cast<const uint4*>(gu + row * 2 * (long)I + I);
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int idx = min((int)threadIdx.x + j * (int)blockDim.x, nvec - 1);
            gv[b][j] = g4[idx];
            uv[b][j] = u4[idx];
        }
    };
    // alternate reduction buffers (by buffer b): a thread still reading one row's buffer is never overwritten by the
    // next row, whose writes come after the next barrier
    auto process = [&](int b, long row) {
        uint4 r[VPT];
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int idx = threadIdx.x + j * blockDim.x;
            r[j] = make_uint4(0, 0, 0, 0);
            if (idx < nvec) {
                r[j].x = silu_mul_lut2<T>(lut, gv[b][j].x, uv[b][j].x, amax);
                r[j].y = silu_mul_lut2<T>(lut, gv[b][j].y, uv[b][j].y, amax);
                r[j].z = silu_mul_lut2<T>(lut, gv[b][j].z, uv[b][j].z, amax);
                r[j].w = silu_mul_lut2<T>(lut, gv[b][j].w, uv[b][j].w, amax);
            }
        }
        amax = block_max(amax, red + 16 * b);
        const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        if (threadIdx.x == 0) scales[row] = amax / 127.0f;
        uint2* qo = reinterpret_cast<uint2*>(q + row * (long)I);
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int idx = threadIdx.x + j * blockDim.x;
            if (idx < nvec) {
                const uint32_t w[4] = {r[j].x, r[j].y, r[j].z, r[j].w};
                int bq[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    bq[2 * e] = q8(lo_half(w[e], T{}) * inv);
                    bq[2 * e + 1] = q8(hi_half(w[e], T{}) * inv);
                }
                qo[idx] = make_uint2(pack4(bq[0], bq[1], bq[2], bq[3]), pack4(bq[4], bq[5], bq[6], bq[7]));
            }
        }
    };
    // rows b, b + G, ...: peeled so that no prefetch sits under a condition
    const long G = gridDim.x, r0 = blockIdx.x;
    const int cnt = (int)((M - 1 - r0) / G) + 1;
    load(0, r0);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));            // this wavefront's part of the table has landed
    __syncthreads();                                      // the whole table is in LDS
    int k = 0;
    for (; k + 2 < cnt; k += 2) {
        load(1, r0 + (k + 1) * G);
        process(0, r0 + k * G);
        load(0, r0 + (k + 2) * G);
        process(1, r0 + (k + 1) * G);
    }
    if (k + 1 < cnt) {
        load(1, r0 + (k + 1) * G);
        process(0, r0 + k * G);
        process(1, r0 + (k + 1) * G);
    } else {
        process(0, r0 + k * G);
    }
}

// ---- residual add + RMSNorm + per-token quant ----------------------------------------------------------------------
constexpr int MAX_VPT_NORM = 6;                          // input + residual in registers: 8 VGPRs a vector

__device__ __forceinline__ double block_sum_d(double v, double* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);   // butterfly: every lane holds the sum
    const int nw = blockDim.x >> 6;
    if (nw == 1) return v;
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    double t = red[0];
    for (int i = 1; i < nw; ++i) t += red[i];                            // fixed order: identical in every thread
    return t;
}

// One block per row, the row (input and residual) in registers.  RES: a residual is added and updated in place.
template <typename T, int VPT, bool RES>
__global__ void __launch_bounds__(1024) rms_norm_quant_kernel(const uint16_t* __restrict__ x, uint16_t* __restrict__ res,
                                                              const uint16_t* __restrict__ w,
                                                              const float* __restrict__ ub, float eps,
                                                              int8_t* __restrict__ q, float* __restrict__ scales,
                                                              int K) {
    __shared__ double redd[16];
    __shared__ float red[16];
    const long row = blockIdx.x;
    const uint4* xr = reinterpret_cast<const uint4*>(x + row * (long)K);
    uint4* rr = reinterpret_cast<uint4*>(res + row * (long)K);          // used only with RES
    const uint4* w4 = reinterpret_cast<const uint4*>(w);
    const int nvec = K >> 3;
    uint4 xv[VPT], rv[VPT], wv[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        // every load unconditional (an in-bounds vector past the row's end, masked where used): a conditional load
        // made the compiler wait for the row and the residual before issuing the norm weights' load
        const int idx = min((int)threadIdx.x + j * (int)blockDim.x, nvec - 1);
        xv[j] = xr[idx];
        rv[j] = RES ? rr[idx] : make_uint4(0, 0, 0, 0);
        wv[j] = w4[idx];
    }
    auto sum_at = [&](int j, int e, bool hi) -> float {                  // s = float(x) + float(r), one rounding
        const uint32_t xw = e == 0 ? xv[j].x : e == 1 ? xv[j].y : e == 2 ? xv[j].z : xv[j].w;
        const float xf = hi ? hi_half(xw, T{}) : lo_half(xw, T{});
        if constexpr (!RES) return xf;
        const uint32_t rw = e == 0 ? rv[j].x : e == 1 ? rv[j].y : e == 2 ? rv[j].z : rv[j].w;
        return xf + (hi ? hi_half(rw, T{}) : lo_half(rw, T{}));
    };
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int idx = threadIdx.x + j * blockDim.x;
        if (idx < nvec) {
            uint32_t o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float lo = sum_at(j, e, false), hi = sum_at(j, e, true);
                ss += (double)lo * (double)lo;
                ss += (double)hi * (double)hi;
                o[e] = (uint32_t)from_float<T>(lo) | ((uint32_t)from_float<T>(hi) << 16);
            }
            if constexpr (RES) rr[idx] = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
    ss = block_sum_d(ss, redd);
    const float ms = (float)(ss / (double)K);
    const float rms = 1.0f / sqrtf(ms + eps);                            // IEEE sqrt and division

    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int idx = threadIdx.x + j * blockDim.x;
        uint32_t o[4] = {0, 0, 0, 0};
        if (idx < nvec) {
            const uint32_t ww[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint16_t yb[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float t = sum_at(j, e, h == 1) * rms;
                    const float n = to_float(T{from_float<T>(t)});
                    const float p = n * (h ? hi_half(ww[e], T{}) : lo_half(ww[e], T{}));   // exact product
                    yb[h] = from_float<T>(p);
                    amax = __builtin_fmaxf(amax, __builtin_fabsf(to_float(T{yb[h]})));
                }
                o[e] = (uint32_t)yb[0] | ((uint32_t)yb[1] << 16);
            }
        }
        xv[j] = make_uint4(o[0], o[1], o[2], o[3]);                    // y replaces x
    }
    amax = block_max(amax, red);
    const float a = ub && *ub < amax ? *ub : amax;
    float scale = a / 127.0f;
    if (!(scale >= FLT_EPSILON)) scale = FLT_EPSILON;
    const float inv = 1.0f / scale;
    if (threadIdx.x == 0) scales[row] = scale;
    uint2* qo = reinterpret_cast<uint2*>(q + row * (long)K);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int idx = threadIdx.x + j * blockDim.x;
        if (idx < nvec) {
            const uint32_t yw[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
            int b[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                b[2 * e] = q8(lo_half(yw[e], T{}) * inv);
                b[2 * e + 1] = q8(hi_half(yw[e], T{}) * inv);
            }
            qo[idx] = make_uint2(pack4(b[0], b[1], b[2], b[3]), pack4(b[4], b[5], b[6], b[7]));
        }
    }
}

// Any K and alignment: three passes over the row (input and residual re-read from L2), the residual written last.
template <typename T>
__global__ void __launch_bounds__(256) rms_norm_quant_any_kernel(const uint16_t* __restrict__ x,
                                                                 uint16_t* __restrict__ res,
                                                                 const uint16_t* __restrict__ w,
                                                                 const float* __restrict__ ub, float eps,
                                                                 int8_t* __restrict__ q, float* __restrict__ scales,
                                                                 int K) {
    __shared__ double redd[16];
    __shared__ float red[16];
    const long row = blockIdx.x;
    const uint16_t* xr = x + row * (long)K;
    uint16_t* rr = res ? res + row * (long)K : nullptr;
    auto sum_at = [&](int k) -> float {
        const float xf = to_float(T{xr[k]});
        return rr ? xf + to_float(T{rr[k]}) : xf;
    };
    double ss = 0.0;
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        const float v = sum_at(k);
        ss += (double)v * (double)v;
    }
    ss = block_sum_d(ss, redd);
    const float ms = (float)(ss / (double)K);
    const float rms = 1.0f / sqrtf(ms + eps);
    auto y_at = [&](int k) -> float {
        const float n = to_float(T{from_float<T>(sum_at(k) * rms)});
        return to_float(T{from_float<T>(n * to_float(T{w[k]}))});
    };
    float amax = 0.0f;
    for (int k = threadIdx.x; k < K; k += blockDim.x) amax = __builtin_fmaxf(amax, __builtin_fabsf(y_at(k)));
    amax = block_max(amax, red);
    const float a = ub && *ub < amax ? *ub : amax;
    float scale = a / 127.0f;
    if (!(scale >= FLT_EPSILON)) scale = FLT_EPSILON;
    const float inv = 1.0f / scale;
    if (threadIdx.x == 0) scales[row] = scale;
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        q[row * (long)K + k] = (int8_t)q8(y_at(k) * inv);
        if (rr) rr[k] = from_float<T>(sum_at(k));       // after every read of this element's residual
    }
}

// float32 -> 16-bit rounding of the epilogues and the SiLU kernel (test export).
template <typename T>
__global__ void round16_kernel(const float* __restrict__ x, uint16_t* __restrict__ out, long n) {
    const long i = blockIdx.x * (long)blockDim.x + threadIdx.x;
    if (i < n) out[i] = from_float<T>(x[i]);
}

// ---- launch helpers ------------------------------------------------------------------------------------------------
// Threads per row: the smallest power-of-two multiple of 64 (<= 1024) that keeps the row within max_vpt vectors.
static int pick_threads(int nvec, int max_vpt, int* vpt) {
    int t = 64;
    while (t < 1024 && (nvec + t - 1) / t > max_vpt) t <<= 1;
    *vpt = (nvec + t - 1) / t;
    if (*vpt < 1) *vpt = 1;
    return t;
}


// Fewer rows than CUs: as many threads per row as it has vectors (up to 1024), so that each thread's serial share
// of the row is small (M = 1, K = 5120: per-token quant 2.9 -> 2.2 us, RMSNorm + quant 4.5 -> 3.8 us).
static int pick_threads_m(int nvec, int max_vpt, int* vpt, int M) {
    if (M >= 256) return pick_threads(nvec, max_vpt, vpt);
    int t = (nvec + 63) / 64 * 64;
    if (t < 64) t = 64;                                   // nvec = 0 (K < 8): the any-K kernel takes the row
    if (t > 1024) t = 1024;
    *vpt = (nvec + t - 1) / t;
    return t;
}
template <typename T, int VPT>
static void launch_ptq(const uint16_t* x, int8_t* q, float* s, int M, int K, long ldx, int threads, hipStream_t st) {
    per_token_quant_kernel<T, VPT><<<M, threads, 0, st>>>(x, q, s, K, ldx);
}

template <typename T>
static int run_ptq(const void* x, void* q, void* s, int M, int K, long ldx, hipStream_t st) {
    const uint16_t* xp = static_cast<const uint16_t*>(x);
    int8_t* qp = static_cast<int8_t*>(q);
    float* sp = static_cast<float*>(s);
    const bool vec_ok = (K % 8 == 0) && (ldx % 8 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)q % 8 == 0);
    int vpt = 0;
    const int threads = pick_threads_m(K / 8, MAX_VPT_QUANT, &vpt, M);
    if (!vec_ok || vpt > MAX_VPT_QUANT) {
        per_token_quant_any_kernel<T><<<M, 256, 0, st>>>(xp, qp, sp, K, ldx);
        return 0;
    }
    switch (vpt) {
#define W8_CASE(V) case V: launch_ptq<T, V>(xp, qp, sp, M, K, ldx, threads, st); break;
        W8_CASE(1) W8_CASE(2) W8_CASE(3) W8_CASE(4) W8_CASE(5) W8_CASE(6) W8_CASE(7) W8_CASE(8)
        W8_CASE(9) W8_CASE(10) W8_CASE(11) W8_CASE(12) W8_CASE(13) W8_CASE(14) W8_CASE(15) W8_CASE(16)
#undef W8_CASE
        default: return -1;
    }
    return 0;
}

// The table kernel takes every row of up to LUT_MAX_VPT vectors per thread; longer rows take the direct kernel.  The
// table kernel is as fast or faster at every M (M=1 7.3 -> 5.5 us, M=511 15.2 -> 11.1 us, M=4096 -9% at I = 17408).
constexpr int LUT_MAX_VPT = 5;                            // I <= 40960: two row buffers in registers, no spills
enum : int { SMQ_ANY = 0, SMQ_DIRECT = 1, SMQ_TABLE = 2 };


template <typename T, int VPT>
static void launch_smq_lut(const uint16_t* gp, int8_t* qp, float* sp, int M, int I, int threads, hipStream_t st) {
    const void* kern = reinterpret_cast<const void*>(&silu_mul_quant_lut_kernel<T, VPT>);
    static const hipError_t attr = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, LUT_LDS_BYTES);
    (void)attr;
    const int grid = M < cu_count() ? M : cu_count();
    silu_mul_quant_lut_kernel<T, VPT><<<grid, threads, LUT_LDS_BYTES, st>>>(gp, qp, sp, M, I);
}

template <typename T>
static int run_smq(const void* gu, void* q, void* s, int M, int I, hipStream_t st, int path = SMQ_ANY) {
    const int nvec = I / 8, lvpt = (nvec + 1023) / 1024;
    const bool table_ok = lvpt <= LUT_MAX_VPT && path != SMQ_DIRECT;
    if (path == SMQ_TABLE && !table_ok) return 1;
    if (table_ok) {
        const int threads = ((nvec + lvpt - 1) / lvpt + 63) / 64 * 64;
        const uint16_t* gp = static_cast<const uint16_t*>(gu);
        int8_t* qp = static_cast<int8_t*>(q);
        float* sp = static_cast<float*>(s);
        switch (lvpt) {
#define W8_CASE(V) case V: launch_smq_lut<T, V>(gp, qp, sp, M, I, threads, st); break;
            W8_CASE(1) W8_CASE(2) W8_CASE(3) W8_CASE(4) W8_CASE(5)
#undef W8_CASE
            default: return 1;
        }
        return 0;
    }
    int vpt = 0;
    const int threads = pick_threads(I / 8, MAX_VPT_SILU, &vpt);
    if (vpt > MAX_VPT_SILU) return 1;
    const uint16_t* gp = static_cast<const uint16_t*>(gu);
    int8_t* qp = static_cast<int8_t*>(q);
    float* sp = static_cast<float*>(s);
    switch (vpt) {
#define W8_CASE(V) case V: silu_mul_quant_kernel<T, V><<<M, threads, 0, st>>>(gp, qp, sp, I); break;
        W8_CASE(1) W8_CASE(2) W8_CASE(3) W8_CASE(4) W8_CASE(5) W8_CASE(6) W8_CASE(7) W8_CASE(8)
#undef W8_CASE
        default: return 1;
    }
    return 0;
}

template <typename T, bool RES>
static int run_rnq_res(const void* x, void* res, const void* w, const float* ub, float eps, void* q, void* s, int M,
                       int K, hipStream_t st) {
    const uint16_t* xp = static_cast<const uint16_t*>(x);
    uint16_t* rp = static_cast<uint16_t*>(res);
    const uint16_t* wp = static_cast<const uint16_t*>(w);
    int8_t* qp = static_cast<int8_t*>(q);
    float* sp = static_cast<float*>(s);
    int vpt = 0;
    const int threads = pick_threads_m(K / 8, MAX_VPT_NORM, &vpt, M);
    switch (vpt) {
#define W8_CASE(V) case V: rms_norm_quant_kernel<T, V, RES><<<M, threads, 0, st>>>(xp, rp, wp, ub, eps, qp, sp, K); break;
        W8_CASE(1) W8_CASE(2) W8_CASE(3) W8_CASE(4) W8_CASE(5) W8_CASE(6)
#undef W8_CASE
        default: return -1;
    }
    return 0;
}

template <typename T>
static int run_rnq(const void* x, void* res, const void* w, const float* ub, float eps, void* q, void* s, int M, int K,
                   hipStream_t st) {
    const bool vec_ok = K % 8 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)res % 16 == 0 && (uintptr_t)w % 16 == 0 &&
                        (uintptr_t)q % 8 == 0 && (K / 8 + 1023) / 1024 <= MAX_VPT_NORM;
    if (!vec_ok) {
        rms_norm_quant_any_kernel<T><<<M, 256, 0, st>>>(static_cast<const uint16_t*>(x), static_cast<uint16_t*>(res),
                                                         static_cast<const uint16_t*>(w), ub, eps,
                                                         static_cast<int8_t*>(q), static_cast<float*>(s), K);
        return 0;
    }
    return res ? run_rnq_res<T, true>(x, res, w, ub, eps, q, s, M, K, st)
               : run_rnq_res<T, false>(x, res, w, ub, eps, q, s, M, K, st);
}

}  // namespace w8

using namespace w8;

// Dynamic per-token int8 quantization (the eager vllm._custom_ops.scaled_int8_quant the reference leaves to vLLM,
// vllm_turing/quantfuse.py:35-39).  x: [M, K] fp16 (dtype 0) or bf16 (dtype 1) with row stride ldx elements;
// q: [M, K] int8 contiguous; scales: [M] float32.  Returns 0, -1 on bad arguments, or the HIP launch error.
extern "C" int per_token_quant(const void* x, void* q, void* scales, int M, int K, long ldx, int dtype, void* stream) {
    if (M < 0 || K < 1 || ldx < K || (dtype != DT_F16 && dtype != DT_BF16) || !x || !q || !scales) return -1;
    if (M == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    const int rc = dtype == DT_F16 ? run_ptq<f16>(x, q, scales, M, K, ldx, st) : run_ptq<bf16>(x, q, scales, M, K, ldx, st);
    if (rc != 0) return rc;
    return (int)hipGetLastError();
}

static int smq_entry(const void* gu, void* q, void* scales, int M, int I, int dtype, void* stream, int path = SMQ_ANY) {
    if (I < 8 || I % 8 != 0 || M < 0) return 1;
    if ((uintptr_t)gu % 16 != 0 || (uintptr_t)q % 8 != 0) return 1;
    if (M == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    const int rc = dtype == DT_F16 ? run_smq<f16>(gu, q, scales, M, I, st, path)
                                   : run_smq<bf16>(gu, q, scales, M, I, st, path);
    if (rc != 0) return rc;
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

// SiLU(gate) * up + per-row int8 quantization, fp16 (csrc/silu_quant.cu:71-77: same arguments and return codes:
// 0 ok, 1 bad I, 2 launch error).  gu: [M, 2I] fp16, q: [M, I] int8, scales: [M] float32.  I % 8 == 0, I <= 65536.
extern "C" int silu_mul_quant(const void* gu, void* q, void* scales, int M, int I, void* stream) {
    return smq_entry(gu, q, scales, M, I, DT_F16, stream);
}

// The same for bf16 activations (no counterpart kernel in the reference, whose kernel is fp16 only; the arithmetic is
// vLLM's bf16 silu_and_mul followed by the same quantization).
extern "C" int silu_mul_quant_bf16(const void* gu, void* q, void* scales, int M, int I, void* stream) {
    return smq_entry(gu, q, scales, M, I, DT_BF16, stream);
}

// Test export: silu_mul_quant / silu_mul_quant_bf16 (dtype 0 / 1) through one kernel: path 1 the direct kernel, 2 the
// table kernel (returns 1 where it does not apply: I > 40960).
extern "C" int silu_mul_quant_path(const void* gu, void* q, void* scales, int M, int I, int dtype, int path,
                                   void* stream) {
    if ((dtype != DT_F16 && dtype != DT_BF16) || (path != SMQ_DIRECT && path != SMQ_TABLE)) return 1;
    return smq_entry(gu, q, scales, M, I, dtype, stream, path);
}

// Test export: silu of all 65,536 input patterns into out[65536] (uint16 bit patterns): dtype 0 / 1 computed by the
// device (fp16 / bf16), 2 / 3 the compiled-in table the SiLU kernel looks up (fp16 / bf16).
extern "C" int silu_table(void* out, int dtype, void* stream) {
    if (!out || dtype < 0 || dtype > 3) return -1;
    hipStream_t st = (hipStream_t)stream;
    const int table = dtype >= 2, dt = dtype & 1;
    if (dt == DT_F16) silu_table_kernel<f16><<<256, 256, 0, st>>>(static_cast<uint16_t*>(out), table);
    else silu_table_kernel<bf16><<<256, 256, 0, st>>>(static_cast<uint16_t*>(out), table);
    return (int)hipGetLastError();
}

// Test export: out[i] = the device's round-to-nearest-even of x[i] to fp16 (dtype 0) or bf16 (dtype 1), as the
// epilogues and the SiLU kernel round, for n values.
extern "C" int f32_to_16(const void* x, void* out, long n, int dtype, void* stream) {
    if (!x || !out || n < 0 || n > (1L << 40) || (dtype != DT_F16 && dtype != DT_BF16)) return -1;
    if (n == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    const long blocks = (n + 255) / 256;
    if (dtype == DT_F16) round16_kernel<f16><<<blocks, 256, 0, st>>>(static_cast<const float*>(x), static_cast<uint16_t*>(out), n);
    else round16_kernel<bf16><<<blocks, 256, 0, st>>>(static_cast<const float*>(x), static_cast<uint16_t*>(out), n);
    return (int)hipGetLastError();
}

// Residual add + RMSNorm + dynamic per-token int8 quantization: vLLM's rms_norm_dynamic_per_token_quant(input, weight,
// epsilon, int8, scale_ub, residual) as the reference's MLP tail calls it (vllm_turing/tailoverlap.py:145).
// x: [M, K] fp16 (dtype 0) or bf16 (dtype 1), row-major; residual: [M, K] of the same type, updated in place to
// RN(x + residual), or null; weight: [K]; scale_ub: one float32 upper bound on the row absmax, or null; q: [M, K]
// int8; scales: [M] float32.  Returns 0, -1 on bad arguments, or the HIP launch error.
extern "C" int rms_norm_quant(const void* x, void* residual, const void* weight, const void* scale_ub, float eps,
                              void* q, void* scales, int M, int K, int dtype, void* stream) {
    if (M < 0 || K < 1 || (dtype != DT_F16 && dtype != DT_BF16) || !x || !weight || !q || !scales || !(eps >= 0.0f))
        return -1;
    if (M == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    const float* ub = static_cast<const float*>(scale_ub);
    const int rc = dtype == DT_F16 ? run_rnq<f16>(x, residual, weight, ub, eps, q, scales, M, K, st)
                                   : run_rnq<bf16>(x, residual, weight, ub, eps, q, scales, M, K, st);
    if (rc != 0) return rc;
    return (int)hipGetLastError();
}
