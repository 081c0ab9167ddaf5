// W8A8 int8 x int8 -> int32 matrix products with the fused scale epilogue, for gfx950 (CDNA4).
//
//   out[m, n] = RN_T( epilogue( acc[m, n], sa[m], sw[n], bias[n] ) ),  acc[m, n] = sum_k a[m, k] * w[n, k]
//
// a: [M, K] int8 row-major (per-token quantized activations); w: [N, K] int8 row-major (the weight as vLLM stores
// it, passed to cutlass_scaled_mm as its [K, N] stride-(1, K) view); sa: float32 [M] or [1]; sw: float32 [N] or [1];
// bias: [N] of the output type or null; out: [M, N] fp16 or bf16.
//
// Six kernels on the path (and two helpers: hbm_read_kernel, the M = 1 GEMV's weight stream without its math, the
// read ceiling the benchmark reports; clear_ints_kernel, which zeroes the allocation-free entry's tile counters):
//  * gemv_dot4_kernel, M = 1 and K <= 17408, M = 2, 3 and K <= 8192, M = 4, 5 and K <= 5120 (decode): weight-streaming
//    through the VALU: each wavefront instruction reads 1 KB contiguous of one weight row, v_dot4_i32_i8 against
//    activations held in registers, wavefront reduction with DPP / ds_swizzle.  Small-M epilogue chain
//    (csrc/w8a8_gemv.cu:91).  Two fused forms: QX quantizes 16-bit activations per token in each workgroup's LDS
//    first (w8a8_gemv_quant), SILU pairs each gate row with its up row and writes silu(g) * u (w8a8_gemv_silu).
//  * stream_lds_kernel, the rest of M <= 32 (decode, speculative verify), and passes of up to 64 rows for 33..128 rows
//    against small N: weight-streaming and HBM-bound.  A workgroup owns one to three 16-row weight tiles; its 4 (or 2)
//    wavefronts take interleaved 128-byte K steps, each through a private LDS ring filled by direct-to-LDS loads of
//    1 KB (8 rows x 128 contiguous bytes each), and feed v_mfma_i32_16x16x64_i8 with the weights as the A operand and
//    up to 16 activation rows per MFMA as the B operand.  The K slices of a tile meet in LDS.  The launch picks the
//    wavefronts, ring depth and tiles per workgroup from how the tiles fill the resident slots.  Small-M epilogue
//    chain (the large-M one when it serves the prefill entry).
//  * w8a16_dot_kernel (the int8 LM head: fp16 / bf16 activations, M <= 2): the dot4 kernel's weight stream, each
//    weight widened exactly to 16-bit pairs for v_dot2_f32_{f16,bf16}; float32 sums.
//  * w8a16_kernel (the int8 LM head, the rest of M <= 32): the LDS-ring weight stream (two or three 16-row tiles per
//    workgroup sharing each activation fragment) with each int8 fragment widened to fp16 / bf16 in registers for
//    v_mfma_f32_16x16x32_{f16,bf16}; float32 sums.
//  * gemm_pp_kernel, M > 32 (prefill), the main configuration: MFMA-bound.  256 x 256 output tiles, 8 wavefronts of
//    128 x 64 (each a 4 x 2 grid of v_mfma_i32_32x32x32_i8) in two groups of four, one of each per SIMD, that
//    alternate between a compute phase (the MFMAs of one K stage from registers) and a memory phase (all operand
//    fragments of the next stage from LDS); 128-byte K stages loaded straight from HBM into LDS (buffer_load ... lds),
//    double-buffered (128 KB), with an XOR swizzle of the 16-byte chunks that keeps ds_read_b128 conflict-free;
//    workgroups remapped so the tiles resident on one XCD share A rows and W rows in that XCD's L2.  With a
//    workspace, a last partial round of tiles runs as K pieces whose int32 partial sums meet in it (split_exchange).
//    The epilogue goes through LDS so that every global store writes whole lines, non-temporally.  Large-M epilogue
//    (csrc/w8a8_big.cu:26-35).
//  * gemm_kernel, the other prefill configurations: where the 256 x 256 tiles leave a last partial round over the
//    CUs and no K split is taken, that round runs as 128 x 128 quarter tiles (4 wavefronts of 64 x 64: two
//    workgroups per CU, or one with 4 K stages in flight where they fit in one round), so it spreads over the whole
//    chip; 33..128 rows (and 129..256 against small N) run on 64 x 128 or 64 x 64 tiles with 4 K stages in flight,
//    the 64 x 64 tiles of 33..64 rows as two K pieces where those fit two workgroups per CU.
//
// The kernels use the freedom that an integer dot product does not depend on the order of k: each lane feeds the
// MFMA the same permutation of k on its A and B operands (the dot4 kernel pairs weight and activation chunks the
// same way), so every operand is a contiguous 16-byte vector.
// Integer accumulation is exact (|acc| < 2^31 for K < 131072), so split-K order and tile order are free and the int32
// results are bit-exact.
#include <type_traits>

#include "common.h"
#include "../../include/w8a8_mi355.h"

namespace w8 {

enum : int { EPI_SMALL = 0, EPI_LARGE = 1, EPI_LARGE_BIAS = 2, EPI_I32 = 3 };

// ---------------------------------------------------------------------------------------------------------------------
// output write of one element, per epilogue
// ---------------------------------------------------------------------------------------------------------------------
template <typename T, int EPI>
__device__ __forceinline__ void store_out(void* out, long idx, int acc, const float* sa, int m, const float* sw, int n,
                                          const uint16_t* bias) {
    if constexpr (EPI == EPI_I32) {
        static_cast<int*>(out)[idx] = acc;                // no scale is read: sa / sw / bias may be null
    } else {
        const float sam = sa[m], swn = sw[n];
        float r;
        if constexpr (EPI == EPI_SMALL) r = epi_small(acc, sam, swn, bias ? to_float(T{bias[n]}) : 0.0f);
        else if constexpr (EPI == EPI_LARGE) r = epi_large(acc, sam, swn);
        else r = epi_large_bias(acc, sam, swn, to_float(T{bias[n]}));
        static_cast<uint16_t*>(out)[idx] = from_float<T>(r);
    }
}

// Weight loads: read once, so non-temporal (global_load_dwordx4 ... nt) by default.
template <bool NT>
__device__ __forceinline__ v4i wload(const int8_t* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
    else return *reinterpret_cast<const v4i*>(p);
}

// Four 16-bit zeros: the bias operand of a 4-column group without bias.
__device__ __align__(16) const uint16_t g_zero4[4] = {0, 0, 0, 0};
// A 16-bit zero in device memory: the bias operand of a row without bias, so that the bias load is unconditional.
__device__ const uint16_t g_zero16 = 0;
// A value loaded through a global-address-space pointer: a load through a pointer the compiler cannot place (such as
// a select between a kernel argument and g_zero16) becomes a FLAT load, which counts on two counters and completes
// out of order, and then every wait for vector memory drains all loads in flight.
template <typename V>
__device__ __forceinline__ V gload(const void* p) {
    return *(const __attribute__((address_space(1))) V*)p;
}

// Output write of one element as store_out, with the scales and bias already in registers.
template <typename T, int EPI>
__device__ __forceinline__ void store_pre(void* out, long idx, int acc, float sam, float swn, float bn) {
    if constexpr (EPI == EPI_I32) {
        static_cast<int*>(out)[idx] = acc;
    } else {
        float r;
        if constexpr (EPI == EPI_SMALL) r = epi_small(acc, sam, swn, bn);
        else if constexpr (EPI == EPI_LARGE) r = epi_large(acc, sam, swn);
        else r = epi_large_bias(acc, sam, swn, bn);
        static_cast<uint16_t*>(out)[idx] = from_float<T>(r);
    }
}

// ---------------------------------------------------------------------------------------------------------------------
// gemv_dot4_kernel: M <= 5 activation rows, weights streamed once through the VALU
// ---------------------------------------------------------------------------------------------------------------------
// Every wavefront instruction reads 1 KB of one weight row (64 lanes x 16 contiguous bytes); lane l owns the 16-byte
// chunks l, l + 64, ... of every row (CH of them), and keeps the matching activation chunks of all M rows in
// registers for the whole kernel.  Rows are grid-strided over the wavefronts, R rows per iteration with the next
// iteration's loads issued before this one's v_dot4 math (double buffering).  Each row's per-lane partial sums are
// reduced across the wavefront with DPP row operations, ds_swizzle and readlane.
// QX: the activations arrive as fp16 / bf16 rows x (row stride ldx elements, the output type) and every workgroup
// quantizes them into LDS before its first row's math, with per_token_quant's arithmetic (absmax over the row; scale
// = absmax / 127; q = clamp(rint(x * (127 / absmax)))), while its wavefronts' first weight rows are already being
// loaded (each workgroup reads the row once: per wavefront it cost ~140 MB of L2 reads at N = 5120); workgroup 0 also
// writes the int8 rows to xq and the scales to xs.
// SILU: the weights are a gate_up projection of 2N rows (gate rows 0..N-1, up rows N..2N-1) and a row group is the
// pair (p, p + N) (R = 2); instead of the two outputs the kernel writes out[m, p] = silu(g) * u in 16 bits, with g and
// u rounded as the GEMV writes them and the product as silu_mul_quant forms it before quantizing
// (vllm_turing/csrc/silu_quant.cu:39), so the decode MLP needs no separate SiLU kernel.
// DEF (the one-wavefront grid of M <= 2, whose launch gives every wavefront at most DEF = 3 row groups): the outputs
// stay in registers and are stored after the last group.  An output store between two groups' loads keeps the
// compiler from counting the loads still in flight (stores and loads complete out of order against each other), so
// its wait before each group's math drained every load, and a wavefront had one group in flight instead of two.
constexpr int QX_THREADS = 256;                          // threads of a workgroup of the fused-quant GEMV
template <typename T, int M, int CH, int R, int EPI, bool NT = true, bool QX = false, bool SILU = false, int DEF = 0>
__global__ void __launch_bounds__(256) gemv_dot4_kernel(const int8_t* __restrict__ a, const int8_t* __restrict__ w,
                                                        const float* __restrict__ sa, const float* __restrict__ sw,
                                                        const uint16_t* __restrict__ bias, void* __restrict__ out,
                                                        int N, int K, int sa_rows, int sw_rows,
                                                        const uint16_t* __restrict__ x = nullptr, long ldx = 0,
                                                        int8_t* __restrict__ xq = nullptr,
                                                        float* __restrict__ xs = nullptr) {
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * (blockDim.x >> 6);
    const int wid = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int K16 = K >> 4;
    static_assert(!SILU || (R == 2 && EPI == EPI_SMALL && !QX), "gate and up rows of one pair, small-M epilogue");
    const v4i z = {0, 0, 0, 0};
    v4i av[M][CH];
    float sam[M];                                        // row scales (none are read for the int32 output)
    v4i wb[2][R][CH];
    float swb[2][R];                                     // the rows' column scale and bias bits, loaded with the row
    uint16_t bb[2][R];
    auto load = [&](int buf, int n0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = SILU ? min(n0, N - 1) + r * N : min(n0 + r * nw, N - 1);
            const int8_t* row = w + (long)n * K;
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int c = lane + 64 * j;
                // no mask on loaded values: a select after the load would make the compiler wait for it right
                // there, serialising the next row's loads with this row's math.  Chunks past K read an in-bounds
                // chunk and meet zero activations; rows past N read row N - 1 and are not stored.
                wb[buf][r][j] = wload<NT>(row + min(c, K16 - 1) * 16);
            }
            // unconditional loads, converted only in finish: a conditional load or a conversion next to it would
            // make the compiler wait for the next row's weights as well
            swb[buf][r] = EPI == EPI_I32 ? 0.0f : sw[sw_rows ? n : 0];
            bb[buf][r] = EPI == EPI_SMALL || EPI == EPI_LARGE_BIAS ? gload<uint16_t>(bias ? bias + n : &g_zero16) : 0;
        }
    };
    // the int32 sums of the row group in buffer buf against every activation row, reduced over the wavefront
    auto sums = [&](int buf, int (&acc)[R][M]) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) {
                int s = 0;
#pragma unroll
                for (int j = 0; j < CH; ++j) {
                    s = __builtin_amdgcn_sdot4(wb[buf][r][j].x, av[m][j].x, s, false);
                    s = __builtin_amdgcn_sdot4(wb[buf][r][j].y, av[m][j].y, s, false);
                    s = __builtin_amdgcn_sdot4(wb[buf][r][j].z, av[m][j].z, s, false);
                    s = __builtin_amdgcn_sdot4(wb[buf][r][j].w, av[m][j].w, s, false);
                }
                acc[r][m] = wave_sum(s);
            }
    };
    auto finish = [&](int buf, int n0) {
        int acc[R][M];
        sums(buf, acc);
        if constexpr (SILU) {                            // lane m writes out[m, n0]
#pragma unroll
            for (int m = 0; m < M; ++m)
                if (lane == m && n0 < N) {
                    const float g = to_float(T{from_float<T>(epi_small(acc[0][m], sam[m], swb[buf][0],
                                                                      to_float(T{bb[buf][0]})))});
                    const float u = to_float(T{from_float<T>(epi_small(acc[1][m], sam[m], swb[buf][1],
                                                                      to_float(T{bb[buf][1]})))});
                    static_cast<uint16_t*>(out)[(long)m * N + n0] = silu_mul<T>(g, u);
                }
            return;
        }
        // lane r * M + m writes output (m, n0 + r * nw)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const int n = n0 + r * nw;
                if (lane == r * M + m && n < N)
                    store_pre<T, EPI>(out, (long)m * N + n, acc[r][m], sam[m], swb[buf][r], to_float(T{bb[buf][r]}));
            }
    };
    // Row groups wid, wid + stride, ... (cnt of them), each computed while the next group's loads are in flight.  The
    // loop is peeled so that no load sits under a condition: then the compiler's wait before a group's math counts
    // the next group's loads as still outstanding instead of waiting for them too.
    const int stride = SILU ? nw : R * nw;
    if constexpr (!QX) {
        if (wid >= N) return;
    }
    const int cnt = wid < N ? (N - 1 - wid) / stride + 1 : 0;
    // rows past N read row N - 1 (see load).  With DEF the first group's loads follow the activations' (conditional)
    // loads instead, so that the wait before its math can count the loads issued after it.
    if constexpr (DEF == 0) load(0, wid);
    if constexpr (QX) {
        // The workgroup quantizes the rows once into LDS (xl: M rows of K int8), each thread 8 values per step:
        // absmax over the row (wavefront max, then across the wavefronts), then the int8 values from a second read
        // of the same (now cached) row; the wavefronts then take their chunks from LDS.  Workgroup 0 also writes
        // the int8 rows and scales out.
        // Each thread loads its whole share of the row (at most XV vectors of 8 values; chunks past the row re-read
        // its last vector, which leaves the maximum unchanged and is not stored) before using any of it, so the
        // prologue waits for one round of loads instead of one per vector and reads the row once.
        extern __shared__ v4i xq_lds[];
        int8_t* xl = reinterpret_cast<int8_t*>(xq_lds);
        float* red = reinterpret_cast<float*>(xl + M * K);   // one float per wavefront
        constexpr int nthr = QX_THREADS, XV = (CH * 128 + QX_THREADS - 1) / QX_THREADS;   // K <= CH * 1024
        const int tid = threadIdx.x, nvec = K >> 3;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const uint4* xr = reinterpret_cast<const uint4*>(x + m * ldx);
            uint4 xv[XV];
#pragma unroll
            for (int i = 0; i < XV; ++i) xv[i] = xr[min(tid + i * nthr, nvec - 1)];
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < XV; ++i) {
                const uint32_t e4[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    amax = __builtin_fmaxf(amax, __builtin_fabsf(lo_half(e4[e], T{})));
                    amax = __builtin_fmaxf(amax, __builtin_fabsf(hi_half(e4[e], T{})));
                }
            }
            amax = wave_max(amax);
            if (lane == 0) red[threadIdx.x >> 6] = amax;
            __syncthreads();
            for (int i = 0; i < (nthr >> 6); ++i) amax = __builtin_fmaxf(amax, red[i]);
            __syncthreads();                             // red is reused by the next row
            const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            sam[m] = amax / 127.0f;
            if (blockIdx.x == 0 && tid == 0) xs[m] = sam[m];
#pragma unroll
            for (int i = 0; i < XV; ++i) {
                const int v = tid + i * nthr;
                if (v >= nvec) break;
                const uint4 u = xv[i];
                const uint32_t e4[4] = {u.x, u.y, u.z, u.w};
                int b[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    b[2 * e] = q8(lo_half(e4[e], T{}) * inv);
                    b[2 * e + 1] = q8(hi_half(e4[e], T{}) * inv);
                }
                const uint2 q2 = make_uint2(pack4(b[0], b[1], b[2], b[3]), pack4(b[4], b[5], b[6], b[7]));
                *reinterpret_cast<uint2*>(xl + m * K + v * 8) = q2;
                if (blockIdx.x == 0) *reinterpret_cast<uint2*>(xq + (long)m * K + v * 8) = q2;
            }
        }
        __syncthreads();
        if (wid >= N) return;                            // after the workgroup's barriers: no rows of its own
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int c = lane + 64 * j;
                av[m][j] = c < K16 ? *reinterpret_cast<const v4i*>(xl + m * K + c * 16) : z;
            }
    } else {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                const int c = lane + 64 * j;
                av[m][j] = c < K16 ? *reinterpret_cast<const v4i*>(a + (long)m * K + c * 16) : z;
            }
#pragma unroll
        for (int m = 0; m < M; ++m) sam[m] = EPI == EPI_I32 ? 0.0f : sa[sa_rows ? m : 0];
    }
    if constexpr (DEF > 0) {
        static_assert(DEF == 3 && !QX && !SILU, "deferred stores: the one-wavefront grid of M <= 2");
        // the value lane r * M + m stores for output (m, n0 + r * nw) of the group in buffer buf
        auto value = [&](int buf) {
            int acc[R][M];
            sums(buf, acc);
            uint32_t v = 0;
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    uint32_t x;
                    if constexpr (EPI == EPI_I32) x = (uint32_t)acc[r][m];
                    else if constexpr (EPI == EPI_SMALL)
                        x = from_float<T>(epi_small(acc[r][m], sam[m], swb[buf][r], to_float(T{bb[buf][r]})));
                    else if constexpr (EPI == EPI_LARGE) x = from_float<T>(epi_large(acc[r][m], sam[m], swb[buf][r]));
                    else x = from_float<T>(epi_large_bias(acc[r][m], sam[m], swb[buf][r], to_float(T{bb[buf][r]})));
                    v = lane == r * M + m ? x : v;
                }
            return v;
        };
        auto put = [&](uint32_t v, int n0) {
            if (lane < R * M) {
                const int r = lane / M, m = lane % M, n = n0 + r * nw;
                if (n < N) {
                    if constexpr (EPI == EPI_I32) static_cast<int*>(out)[(long)m * N + n] = (int)v;
                    else static_cast<uint16_t*>(out)[(long)m * N + n] = (uint16_t)v;
                }
            }
        };
        // groups past cnt load row N - 1 (see load) and are not stored
        load(0, wid);
        load(1, wid + stride);
        __builtin_amdgcn_sched_barrier(0);              // keep the loads ahead of the math
        const uint32_t v0 = value(0);
        load(0, wid + 2 * stride);
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t v1 = value(1);
        const uint32_t v2 = value(0);
        put(v0, wid);
        if (cnt > 1) put(v1, wid + stride);
        if (cnt > 2) put(v2, wid + 2 * stride);
        return;
    }
    int k = 0;
    for (; k + 2 < cnt; k += 2) {
        load(1, wid + (k + 1) * stride);
        finish(0, wid + k * stride);
        load(0, wid + (k + 2) * stride);
        finish(1, wid + (k + 1) * stride);
    }
    if (k + 1 < cnt) {
        load(1, wid + (k + 1) * stride);
        finish(0, wid + k * stride);
        finish(1, wid + (k + 1) * stride);
    } else {
        finish(0, wid + k * stride);
    }
}

// ---------------------------------------------------------------------------------------------------------------------
// gemm_kernel: MFMA 32x32x32 int8 tiles, K stages loaded straight into LDS
// ---------------------------------------------------------------------------------------------------------------------
// The output is cut into 256 x 256 super tiles, rastered in groups of GROUP_M super-tile rows.  A workgroup computes
// either a whole super tile (the main configuration) or one 128 x 128 quarter of one (the small configuration, used
// where the super tiles do not divide evenly over the CUs: the last, partial round of super tiles is done as four
// times as many quarter tiles, which spreads it over the whole chip).
constexpr int SUPER = 256;
constexpr int GROUP_M = 4;                               // super-tile rows per raster group

// WM x WN wavefronts, each owning FM x FN blocks of 32 x 32 outputs (a (32 FM) x (32 FN) wavefront tile), so the
// workgroup tile is BM = 32 WM FM rows by BN = 32 WN FN columns.  K is staged KB bytes per row at a time, NS stages
// rotating in LDS.
template <int WM, int WN, int FM, int FN, int KB, int NS>
struct GemmCfg {
    static constexpr int WAVES = WM * WN, THREADS = 64 * WAVES;
    static constexpr int WTM = 32 * FM, WTN = 32 * FN;   // wavefront tile
    static constexpr int BM = WM * WTM, BN = WN * WTN;   // workgroup tile
    static constexpr int SUB = (SUPER / BM) * (SUPER / BN);   // workgroup tiles per super tile
    static constexpr int CPR = KB / 16;                  // 16-byte chunks per staged row
    static constexpr int RPB = 1024 / KB;                // rows per 1 KB direct-to-LDS block
    static constexpr int STAGE_BYTES = (BM + BN) * KB;
    static constexpr int PITCH = WTN * 2 + 8;            // epilogue LDS row: 16-bit outputs + 8 bytes of padding
    static constexpr int EPI_BYTES = WAVES * WTM * PITCH;
    static constexpr int LDS_BYTES = EPI_BYTES > NS * STAGE_BYTES ? EPI_BYTES : NS * STAGE_BYTES;
    static constexpr int BPWA = BM / RPB / WAVES;        // 1 KB blocks of A per wavefront per stage
    static constexpr int BPWW = BN / RPB / WAVES;        // 1 KB blocks of W per wavefront per stage
    static constexpr int LPW = BPWA + BPWW;              // direct-to-LDS loads per wavefront per stage
    static_assert(BPWA * RPB * WAVES == BM && BPWW * RPB * WAVES == BN, "stages split evenly over the wavefronts");
    static_assert(SUPER % BM == 0 && SUPER % BN == 0, "workgroup tiles divide the super tile");
    static_assert(NS >= 2 && NS <= 6 && LDS_BYTES <= 160 * 1024, "stage configuration");
};

// 16-byte chunk c of a staged LDS row lives at chunk position c ^ swz(row).  A ds_read_b128 phase serves 8 rows
// (128-byte phases) or 16 rows (256-byte phases) reading the same logical chunk; the XOR spreads them over distinct
// 16-byte bank groups in both cases.  With 64-byte rows two rows share a 128-byte bank line (rows of equal parity
// among 8, and rows 4 apart among 16, must differ); with 128-byte rows every row starts at bank 0 (rows among 8 must
// differ; rows 8 apart sit in the same 256-byte half only when of equal parity).  Both depend on row & 15 only.
template <int CPR>
__device__ __forceinline__ int swz(int row) {
    if constexpr (CPR == 4) return ((row >> 1) ^ ((row >> 3) & 1)) & 3;
    else return (row ^ ((row >> 3) & 1)) & 7;
}


// Raw int32 store of one wavefront's (32 FM) x (32 FN) block (test export only): straight from the fragment layout.
template <int FM, int FN>
__device__ __forceinline__ void store_tile_i32(const v16i (&acc)[FM][FN], int* o, int M, int N, int mb, int nb,
                                               int lane) {
    const bool vec = (N & 3) == 0;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int m = mb + i * 32 + (lane & 31);
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = nb + j * 32 + 8 * q + 4 * (lane >> 5);
                if (n >= N) continue;
                const long idx = (long)m * N + n;
                if (vec && n + 3 < N) {
                    *reinterpret_cast<v4i*>(o + idx) =
                        v4i{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                } else {
                    for (int r = 0; r < 4 && n + r < N; ++r) o[idx + r] = acc[i][j][4 * q + r];
                }
            }
        }
    }
}

// Epilogue through LDS: the fragment layout gives each lane 4 consecutive columns of one row, so global stores
// straight from registers write 8-16 byte pieces of many cache lines (measured at a fraction of HBM write bandwidth).
// Instead each wavefront writes its (32 FM) x (32 FN) block of finished 16-bit values into its own LDS region (rows
// padded by 8 bytes: the 8-byte writes of consecutive lanes fall on distinct banks), then reads it back row-major and
// stores whole lines.
template <typename T, int EPI, int FM, int FN, int PITCH>
__device__ __forceinline__ void store_tile_lds(const v16i (&acc)[FM][FN], uint8_t* eb, void* out, const float* sa,
                                               const float* sw, const uint16_t* bias, int M, int N, int sa_rows,
                                               int sw_rows, int mb, int nb, int lane) {
    float sam[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) sam[i] = sa[sa_rows ? min(mb + i * 32 + (lane & 31), M - 1) : 0];
    // per-column scales and bias: with N % 4 == 0, every 4-column group of this wavefront at once, unconditionally
    // (the last group clamped in bounds; its columns past N are never stored), before any is used (~1%)
    const bool has_bias = (EPI == EPI_LARGE_BIAS || EPI == EPI_SMALL) && bias != nullptr;
    const bool vec_cols = (N & 3) == 0 && sw_rows;
    float4 sw4[FN][4];
    uint2 b2[FN][4];
    if (vec_cols) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = min(nb + j * 32 + 8 * q + 4 * (lane >> 5), N - 4);
                sw4[j][q] = *reinterpret_cast<const float4*>(sw + n);
                typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));   // (a HIP uint2 loads as FLAT)
                const u32x2 bv2 = gload<u32x2>(has_bias ? static_cast<const void*>(bias + n) : g_zero4);
                b2[j][q] = make_uint2(bv2.x, bv2.y);
            }
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int nl = j * 32 + 8 * q + 4 * (lane >> 5);
            const int n = nb + nl;
            float swv[4], bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (vec_cols) {
                swv[0] = sw4[j][q].x; swv[1] = sw4[j][q].y; swv[2] = sw4[j][q].z; swv[3] = sw4[j][q].w;
                if (has_bias) {
                    bv[0] = lo_half(b2[j][q].x, T{}); bv[1] = hi_half(b2[j][q].x, T{});
                    bv[2] = lo_half(b2[j][q].y, T{}); bv[3] = hi_half(b2[j][q].y, T{});
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int nn = min(n + r, N - 1);
                    swv[r] = sw[sw_rows ? nn : 0];
                    if (has_bias) bv[r] = to_float(T{bias[nn]});
                }
            }
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int ml = i * 32 + (lane & 31);
                uint16_t h[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int accv = acc[i][j][4 * q + r];
                    float v;
                    if constexpr (EPI == EPI_SMALL) v = epi_small(accv, sam[i], swv[r], bv[r]);
                    else if constexpr (EPI == EPI_LARGE) v = epi_large(accv, sam[i], swv[r]);
                    else v = epi_large_bias(accv, sam[i], swv[r], bv[r]);
                    h[r] = from_float<T>(v);
                }
                *reinterpret_cast<uint2*>(eb + ml * PITCH + nl * 2) =
                    make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
            }
            __builtin_amdgcn_sched_barrier(0);               // no hoisting of the next group's loads
        }
    }
    // the wavefront reads back only what it wrote itself: a wait for its own LDS writes suffices
    __builtin_amdgcn_s_waitcnt(0xc07f);                      // lgkmcnt(0)
    constexpr int LPR = FN * 4;                              // lanes per row: 16 bytes (8 outputs) each
    constexpr int RPI = 64 / LPR;                            // rows per wavefront instruction
    const bool vec = (N & 7) == 0;
    uint16_t* o = static_cast<uint16_t*>(out);
#pragma unroll 4
    for (int it = 0; it < 32 * FM / RPI; ++it) {
        const int rl = it * RPI + lane / LPR, cl = (lane % LPR) * 8;
        const int m = mb + rl, n = nb + cl;
        const uint2 lo = *reinterpret_cast<const uint2*>(eb + rl * PITCH + cl * 2);
        const uint2 hi = *reinterpret_cast<const uint2*>(eb + rl * PITCH + cl * 2 + 8);
        if (m >= M) continue;
        if (vec && n + 7 < N) {
            // streaming (non-temporal) store: every workgroup of a round writes its tile at the same time, and the
            // burst drains faster without allocating the lines in L2 (M 4096 x N 12288 x K 5120: 253 -> 244 us;
            // N = 34816: 726 -> 695 us)
            const v4i v = {(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
            __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(o + (long)m * N + n));
        } else {
            const uint32_t wds[4] = {lo.x, lo.y, hi.x, hi.y};
            for (int e = 0; e < 8 && n + e < N; ++e)
                o[(long)m * N + n + e] = (uint16_t)(e & 1 ? wds[e >> 1] >> 16 : wds[e >> 1] & 0xffff);
        }
    }
}

constexpr int CPOL_NT = 2;                                // cache-policy operand of a buffer load: non-temporal

// Part of one K stage of a wavefront's share of A and W, straight into LDS: its A blocks ja0..ja1 - 1 and W blocks
// jw0..jw1 - 1 (of bpwa and bpww 1 KB blocks per stage), issued alternately.  Block j's lane reads logical chunk ch*[j]
// of its row at offset o*[j]; chunks past the end of K get an offset outside the buffer, which makes the load write
// zeros.  A plain device function (the ranges are constants after inlining): in a template context the host pass
// treats the buffer-descriptor type as a substitution failure and silently drops the kernel's host stub.
__device__ __forceinline__ void dma_part(__amdgpu_buffer_rsrc_t rsa, __amdgpu_buffer_rsrc_t rsw, uint8_t* stage_l,
                                         int a_bytes, const int* oa, const int* cha, int bpwa, int ja0, int ja1,
                                         const int* ow, const int* chw, int bpww, int jw0, int jw1, int k0, int K,
                                         int wave) {
    uint8_t* sa_l = stage_l;
    uint8_t* sw_l = stage_l + a_bytes;
    const int n = max(ja1 - ja0, jw1 - jw0);
#pragma unroll
    for (int i = 0; i < n; ++i) {
        const int ja = ja0 + i, jw = jw0 + i;
        if (ja < ja1) {
            const bool ok = k0 + cha[ja] * 16 < K;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_void*)(sa_l + (wave * bpwa + ja) * 1024), 16,
                                                     ok ? oa[ja] : 0x7fffffff, k0, 0, 0);
        }
        if (jw < jw1) {
            const bool ok = k0 + chw[jw] * 16 < K;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, (lds_void*)(sw_l + (wave * bpww + jw) * 1024), 16,
                                                     ok ? ow[jw] : 0x7fffffff, k0, 0, 0);
        }
    }
}


// One 1 KB direct-to-LDS load: each lane's 16 bytes at voff + k0 of the buffer into dst + 16 * lane (an offset past the
// buffer's end writes zeros).  A plain device function for the reason given at dma_part.
__device__ __forceinline__ void dma_block(__amdgpu_buffer_rsrc_t rs, uint8_t* dst, int voff, int k0) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)dst, 16, voff, k0, 0, 0);
}

// K-split workspace: SPLIT_HEAD_INTS tile counters (zero between calls), then for split tile rt its `splits` slots of
// int32 accumulators, one per K piece, at rt * splits * (slot ints) past the counters.
constexpr int SPLIT_HEAD_INTS = 1024;
constexpr int SPLIT_SLOT_INTS = SUPER * SUPER;           // one super tile of int32 accumulators (256 KB)

// The partial exchange of a K-split tile.  Piece `piece` of tile rt stores this workgroup's int32 accumulators to its
// slot and arrives at the tile's counter; the last to arrive adds the other pieces' slots to its own accumulators
// (integer sums: the result is the same in any order) and sets the counter back to zero.  Returns whether this
// workgroup arrived last, i.e. holds the tile's whole sum and runs the epilogue.  No workgroup waits for another.
// The slots are written and read with agent-coherent accesses (the sc1 form the compiler gives relaxed agent-scope
// atomic stores and loads), so a piece's slot is visible on every XCD once its stores complete, without an L2
// write-back or invalidation (the compiler's agent-scope fences do both, for the whole L2, and made the K split slower
// than no split).  Each wavefront waits for its own stores; the barrier then orders them before the tile's arrival, and
// the last piece's reads after it.  Slot layout: WAVES blocks of FM FN 4 KB, one per wavefront in its fragment order,
// 1 KB per store instruction (lane l at 16 l).
template <int FM, int FN, int WAVES>
__device__ __forceinline__ bool split_exchange(v16i (&acc)[FM][FN], int* ws, int rt, int piece, int splits, int wave,
                                               int lane, int tid) {
    constexpr int WAVE_V4 = FM * FN * 4 * 64;            // 16-byte vectors per wavefront
    constexpr long SLOT_INTS = (long)WAVES * WAVE_V4 * 4;
    constexpr int CPOL_SC1 = 16;
    const __amdgpu_buffer_rsrc_t rsp =
        make_rsrc(ws + SPLIT_HEAD_INTS + (long)rt * splits * SLOT_INTS, (long)splits * SLOT_INTS * 4);
    auto voff = [&](int q, int f, int c) { return ((q * WAVES + wave) * WAVE_V4 + (f * 4 + c) * 64 + lane) * 16; };
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                __builtin_amdgcn_raw_buffer_store_b128(
                    v4i{acc[i][j][4 * c], acc[i][j][4 * c + 1], acc[i][j][4 * c + 2], acc[i][j][4 * c + 3]}, rsp,
                    voff(piece, i * FN + j, c), 0, CPOL_SC1);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __shared__ int last;
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(ws + rt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
    __syncthreads();
    if (!last) return false;
    for (int q = 0; q < splits; ++q) {
        if (q == piece) continue;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const v4i v = __builtin_amdgcn_raw_buffer_load_b128(rsp, voff(q, i * FN + j, c), 0, CPOL_SC1);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][4 * c + e] += v[e];
                }
    }
    if (tid == 0) __hip_atomic_store(ws + rt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// WM x WN wavefronts (main configuration 2 x 4: two per SIMD, so one wavefront's LDS and barrier waits are covered by
// the other's MFMAs).  Workgroup u of the grid computes quarter (or whole) tile u % SUB of super tile t_base + u / SUB.
// KSPLIT (the mid configurations, `splits` K pieces): the grid is every BM x BN tile of the output times `splits`;
// workgroup u (after the XCD remap) runs piece u / T of tile u % T (T tiles, column-major over the BM-row tile rows, so
// that the tile rows of one weight column and the workgroups of one K range sit on one XCD) and meets the other pieces
// in the workspace `ws` (split_exchange); t_base > 0 there selects the uneven two-piece form for the last t_base
// tiles (dispatch order instead of the XCD remap, described where it is mapped).
template <typename T, int EPI, int WM, int WN, int FM, int FN, int KB, int NS, int SPLIT = 0, bool LEAD = false,
          int GM = GROUP_M, bool PRIO = false, bool KSPLIT = false>
__global__ void __launch_bounds__(64 * WM * WN) gemm_kernel(const int8_t* __restrict__ a, const int8_t* __restrict__ w,
                                                            const float* __restrict__ sa, const float* __restrict__ sw,
                                                            const uint16_t* __restrict__ bias, void* __restrict__ out,
                                                            int M, int N, int K, int sa_rows, int sw_rows, int t_base,
                                                            int splits, int* __restrict__ ws) {
    extern __shared__ v4i ldsx[];
    // the wavefront index in a scalar register, so that what derives from it (the LDS block addresses of the
    // direct-to-LDS loads, the wavefront tile origins) is scalar too (M 4096 x N 12288 x K 5120: 228 -> 224 us;
    // M = 512: 40.5 -> 39.5 us)
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    using Cfg = GemmCfg<WM, WN, FM, FN, KB, NS>;
    constexpr int BM = Cfg::BM, BN = Cfg::BN, SUB = Cfg::SUB, WTM = 32 * FM, WTN = 32 * FN;
    constexpr int PITCH = WTN * 2 + 8;

    // XCD-aware remap: hardware places workgroup b on XCD b % 8; give each XCD a contiguous run of tiles (and the
    // SUB quarters of one super tile to the same XCD)
    const int nb = gridDim.x, per = nb >> 3;
    int u = blockIdx.x;
    if (u < per * 8) u = (u & 7) * per + (u >> 3);
    int m0, n0, kst0 = 0, nk = (K + KB - 1) / KB, piece = 0, rt = 0;   // tile origin, first stage and stage count
    if constexpr (KSPLIT) {
        const int TMb = (M + BM - 1) / BM, Tb = TMb * ((N + BN - 1) / BN);
        if (t_base > 0) {
            // uneven two-piece form (splits == 2; t_base = the number of uneven tiles, the last ones), in dispatch
            // order: both halves of each even tile and the long first piece (stages [0, L)) of each uneven tile,
            // which together fill one round of the grid's slots, then the uneven tiles' short pieces, which start on
            // the slots the halves free.  L = h + 5/8 of the rest (32 of 40 stages): 4/8 balances a half and a
            // short piece against a long one on paper; same box, M 64 x N 19456 / 20480 x K 5120, 3/8 32.4 / 34.2
            // us, 4/8 31.9 / 32.8, 5/8 31.5 / 32.1, 6/8 31.4 / 32.1, all within 1% at 272 tiles
            const int b = blockIdx.x, te = Tb - t_base, h = nk / 2, L = h + (nk - h) * 5 / 8;
            if (b < 2 * te) {
                rt = b >> 1;
                piece = b & 1;
            } else {
                const int j = b - 2 * te;
                piece = j >= t_base;
                rt = te + j - piece * t_base;
            }
            const int cut = rt < te ? h : L;
            kst0 = piece ? cut : 0;
            nk = piece ? nk - cut : cut;
        } else {
            piece = u / Tb;
            rt = u % Tb;
            kst0 = piece * nk / splits;
            nk = (piece + 1) * nk / splits - kst0;       // >= 1: the host takes splits <= the stage count
        }
        m0 = (rt % TMb) * BM;
        n0 = (rt / TMb) * BN;
    } else {
        const int TM = (M + SUPER - 1) / SUPER, TN = (N + SUPER - 1) / SUPER;
        const int t = t_base + u / SUB, q = u % SUB;
        const int gsz = GM * TN, grp = t / gsz, first_m = grp * GM;
        const int gm = min(TM - first_m, GM);
        const int tm = first_m + (t % gsz) % gm, tn = (t % gsz) / gm;
        m0 = tm * SUPER + (q / (SUPER / BN)) * BM;
        n0 = tn * SUPER + (q % (SUPER / BN)) * BN;
        if (m0 >= M || n0 >= N) return;                  // a quarter past the edge of the last super tile (uniform)
    }

    // global -> LDS directly (buffer_load_dwordx4 ... lds): one wavefront instruction fills 1 KB of LDS, i.e.
    // 1024 / KB rows of one stage; lane l lands at byte 16 l of it, so it fetches the logical chunk that the swizzle
    // stores at its position.  NS stages rotate in LDS and the loads of stage s + NS - 1 are issued while
    // stage s is computed, so no register holds staged data and the memory latency has NS - 1 stages of MFMA
    // work to hide behind.
    const __amdgpu_buffer_rsrc_t rsa = make_rsrc(a, (long)M * K), rsw = make_rsrc(w, (long)N * K);
    constexpr int CPR = Cfg::CPR, BPWA = Cfg::BPWA, BPWW = Cfg::BPWW;
    const int drow = lane / CPR, pch = lane % CPR;       // row within the 1 KB block; physical chunk position
    int oa[BPWA], cha[BPWA], ow[BPWW], chw[BPWW];        // ch*: the logical chunk the swizzle stores at this position
#pragma unroll
    for (int j = 0; j < BPWA; ++j) {
        const int row = (wave * BPWA + j) * Cfg::RPB + drow;
        cha[j] = pch ^ swz<CPR>(row);
        oa[j] = min(m0 + row, M - 1) * K + cha[j] * 16;
    }
#pragma unroll
    for (int j = 0; j < BPWW; ++j) {
        const int row = (wave * BPWW + j) * Cfg::RPB + drow;
        chw[j] = pch ^ swz<CPR>(row);
        ow[j] = min(n0 + row, N - 1) * K + chw[j] * 16;
    }
    uint8_t* const lbase = reinterpret_cast<uint8_t*>(ldsx);
    auto issue = [&](int stage, int k0) {
        dma_part(rsa, rsw, lbase + stage * Cfg::STAGE_BYTES, BM * KB, oa, cha, BPWA, 0, BPWA, ow, chw, BPWW, 0, BPWW,
                 k0, K, wave);
    };
    auto issue_slice = [&](int stage, int k0, int sl) {  // slice sl of SPLIT
        dma_part(rsa, rsw, lbase + stage * Cfg::STAGE_BYTES, BM * KB, oa, cha, BPWA, sl * BPWA / SPLIT,
                 (sl + 1) * BPWA / SPLIT, ow, chw, BPWW, sl * BPWW / SPLIT, (sl + 1) * BPWW / SPLIT, k0, K, wave);
    };
    static_assert(SPLIT == 0 || (BPWA % SPLIT == 0 && BPWW % SPLIT == 0 && SPLIT <= KB / 32 + (LEAD ? 1 : 0)),
                  "DMA slices");

    const int wm = wave / WN, wn = wave % WN;
    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

    auto compute = [&](int stage, int nstage, int nk0) {    // nk0 < 0: no next stage to load
        const v4i* la = reinterpret_cast<const v4i*>(lbase + stage * Cfg::STAGE_BYTES);
        const v4i* lw = la + BM * CPR;
        v4i fa[2][FM], fw[2][FN];
        auto fload = [&](int sub, int fb) {
            const int cc = 2 * sub + (lane >> 5);        // this lane's 16-byte chunk of the staged row
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int row = wm * WTM + i * 32 + (lane & 31);
                fa[fb][i] = la[row * CPR + (cc ^ swz<CPR>(row))];
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int row = wn * WTN + j * 32 + (lane & 31);
                fw[fb][j] = lw[row * CPR + (cc ^ swz<CPR>(row))];
            }
        };
        constexpr int SUBS = KB / 32;                    // MFMA K steps (32 bytes) per stage
        fload(0, 0);
#pragma unroll
        for (int sub = 0; sub < SUBS; ++sub) {
            if (sub + 1 < SUBS) fload(sub + 1, (sub + 1) & 1);
            // fences keep the next sub-step's fragment reads ahead of this sub-step's MFMAs (left alone, the
            // scheduler re-reads each fragment just before its MFMAs and exposes the LDS latency every time)
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);   // favour the MFMA-issuing wavefront (measured neutral)
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[sub & 1][j], fa[sub & 1][i], acc[i][j], 0, 0,
                                                                      0);
            }
            if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (SPLIT > 0) {                       // next-stage slice sl after this sub-step's MFMAs
                const int sl = sub + (LEAD ? 1 : 0);
                if (sl < SPLIT && nk0 >= 0) issue_slice(nstage, nk0, sl);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    constexpr int WAIT4 = waitcnt_vm(4 * Cfg::LPW), WAIT3 = waitcnt_vm(3 * Cfg::LPW);
    constexpr int WAIT2 = waitcnt_vm(2 * Cfg::LPW), WAIT1 = waitcnt_vm(Cfg::LPW), WAIT0 = waitcnt_vm(0);
    static_assert(4 * Cfg::LPW <= 63, "vmcnt range");
    const int kb0 = kst0 * KB;                           // this workgroup's first K byte
#pragma unroll
    for (int s0 = 0; s0 < NS - 1; ++s0)
        if (s0 < nk) issue(s0, kb0 + s0 * KB);
    for (int kt = 0; kt < nk; ++kt) {
        // this wavefront's loads of stage kt are done once at most the later stages' loads (LPW each) remain
        const int ahead = min(nk - 1 - kt, NS - 2);
        if (NS > 5 && ahead >= 4) __builtin_amdgcn_s_waitcnt(WAIT4);
        else if (NS > 4 && ahead == 3) __builtin_amdgcn_s_waitcnt(WAIT3);
        else if (ahead >= 2) __builtin_amdgcn_s_waitcnt(WAIT2);
        else if (ahead == 1) __builtin_amdgcn_s_waitcnt(WAIT1);
        else __builtin_amdgcn_s_waitcnt(WAIT0);
        // every wavefront's part of stage kt is in LDS (each waited for its own loads above).  A bare s_barrier:
        // __syncthreads() would also wait for the loads of the later stages still in flight.
        __builtin_amdgcn_s_barrier();
        const bool more = kt + NS - 1 < nk;
        if (SPLIT == 0 && more) issue((kt + NS - 1) % NS, kb0 + (kt + NS - 1) * KB);
        if (SPLIT > 0 && LEAD && more) issue_slice((kt + NS - 1) % NS, kb0 + (kt + NS - 1) * KB, 0);
        compute(kt % NS, (kt + NS - 1) % NS, more ? kb0 + (kt + NS - 1) * KB : -1);
    }
    if constexpr (KSPLIT) {
        if (!split_exchange<FM, FN, WM * WN>(acc, ws, rt, piece, splits, wave, lane, tid)) return;
    }

    // D fragment of v_mfma_i32_32x32x32_i8 with the weights as the A operand: lane holds column lane % 32 of the
    // 32 x 32 block (activation row m) and its rows 8 q + 4 (lane / 32) + r, q, r = 0..3 (weight rows n).
    const int mb = m0 + wm * WTM, nbw = n0 + wn * WTN;
    if constexpr (EPI == EPI_I32) {
        store_tile_i32<FM, FN>(acc, static_cast<int*>(out), M, N, mb, nbw, lane);
    } else {
        __syncthreads();                                 // every wavefront is done reading the K stages
        store_tile_lds<T, EPI, FM, FN, PITCH>(acc, reinterpret_cast<uint8_t*>(ldsx) + wave * WTM * PITCH, out, sa, sw,
                                              bias, M, N, sa_rows, sw_rows, mb, nbw, lane);
    }
}

// ---------------------------------------------------------------------------------------------------------------------
// gemm_pp_kernel: the 256 x 256 configuration with its two wavefront groups in alternating roles
// ---------------------------------------------------------------------------------------------------------------------
// The 8 wavefronts of gemm_kernel's main configuration (2 x 4 tiles of 128 x 64, two per SIMD) form two groups of
// four, one wavefront of each per SIMD: group 0 computes rows 0..127 of the tile (activation half A0), group 1 rows
// 128..255 (half A1); both use all 256 weight rows W.  Time is cut into slots separated by workgroup barriers.  In each
// slot one group is in its compute phase (the 32 MFMAs of one K stage, operands in registers) while the other is in its
// memory phase (all 24 operand fragments of its next stage read from LDS into registers, nothing else), so each
// SIMD's matrix pipe is fed by one wavefront while its other wavefront reads LDS.  Group 0 reads stage j in slot 2j
// and computes it in slot 2j + 1; group 1 reads it in slot 2j + 1 and computes it in slot 2j + 2.
//
// Two 64 KB stage buffers (A0 | A1 | W).  A0 of a stage is read only by group 0, A1 only by group 1, W by both, so
// each region of stage j's buffer is released as soon as its readers are done: A0 after slot 2j, A1 and W after slot
// 2j + 1.  The loads of stage j + 2 into that buffer are issued by the computing group, spread between its MFMAs:
//   slot 2j + 1 (group 0): A1 of stage j + 1 and A0 of stage j + 2  (4 + 4 loads of 1 KB per wavefront),
//   slot 2j + 2 (group 1): W of stage j + 2                          (8 loads per wavefront),
// so every region has at least two slots to land, and before each barrier a wavefront waits (vmcnt, exact counts,
// vector memory operations retire in order) for its own loads of the regions read in the next slot.  No group refills
// a region from its memory phase.  Group 0 begins its epilogue while group 1 computes the last stage.
//
// SPLITK: workgroups 0 .. full - 1 take whole super tiles t_base + 0 .. full - 1 as above, and the rest `splits` K
// pieces of each of the next (gridDim.x - full) / splits tiles (workgroup u of that part: piece u / rem of tile
// t_base + full + u % rem, so that the workgroups of one XCD share K ranges).  Piece p runs stages
// [p nk / splits, (p + 1) nk / splits), stores its int32 accumulators to its slot of the workspace and arrives at its
// tile's counter; the last to arrive adds the other pieces' slots to its own accumulators (integer sums: the result is
// the same in any order) and runs the epilogue, then sets the counter back to zero (split_exchange).  No workgroup waits
// for another.
template <typename T, int EPI, bool KFULL, bool SPLITK = false, int GM = GROUP_M, bool PRIO = true>
__global__ void __launch_bounds__(512) gemm_pp_kernel(const int8_t* __restrict__ a, const int8_t* __restrict__ w,
                                                      const float* __restrict__ sa, const float* __restrict__ sw,
                                                      const uint16_t* __restrict__ bias, void* __restrict__ out,
                                                      int M, int N, int K, int sa_rows, int sw_rows, int t_base,
                                                      int splits, int full, int* __restrict__ ws) {
    extern __shared__ v4i ldsx[];
    constexpr int WM = 2, WN = 4, FM = 4, FN = 2, KB = 128, NS = 2;
    using Cfg = GemmCfg<WM, WN, FM, FN, KB, NS>;
    constexpr int BM = Cfg::BM, WTM = 32 * FM, WTN = 32 * FN, PITCH = WTN * 2 + 8, SUBS = KB / 32;
    constexpr int CPR = Cfg::CPR, RPB = Cfg::RPB;        // 8 chunks of 16 bytes per staged row, 8 rows per 1 KB
    static_assert(Cfg::SUB == 1 && WM == 2 && NS == 2 && RPB == 8, "one super tile per workgroup, two groups");
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int grp = wave / WN, gw = wave % WN;           // group, wavefront within the group (== wn)

    // tile mapping of gemm_kernel (XCD-aware remap, raster groups of GM super-tile rows)
    const int TM = (M + SUPER - 1) / SUPER, TN = (N + SUPER - 1) / SUPER;
    // with SPLITK the first `full` workgroups take whole tiles t_base + 0 .. full - 1 (dispatched first, one round
    // over the CUs) and the rest the K pieces of the next tiles, each part remapped within itself
    const bool split_role = SPLITK && (int)blockIdx.x >= full;
    const int base = split_role ? full : 0, cnt = SPLITK ? (split_role ? gridDim.x - full : full) : gridDim.x;
    const int per = cnt >> 3;
    int u = blockIdx.x - base;
    if (u < per * 8) u = (u & 7) * per + (u >> 3);
    int nk = (K + KB - 1) / KB, kst0 = 0, piece = 0, rt = u;   // stages of this workgroup, its first, its K piece
    if (split_role) {
        const int rem = cnt / splits;
        piece = u / rem;
        rt = u % rem;
        kst0 = piece * nk / splits;
        nk = (piece + 1) * nk / splits - kst0;           // >= 1: the host takes splits <= the stage count
    }
    const int t = t_base + base + rt;
    const int gsz = GM * TN, gi = t / gsz, first_m = gi * GM;
    const int gm = min(TM - first_m, GM);
    const int m0 = (first_m + (t % gsz) % gm) * SUPER, n0 = ((t % gsz) / gm) * SUPER;
    if (m0 >= M || n0 >= N) return;                     // uniform over the workgroup, before any barrier

    // This wavefront's 8 loads per pass: group 0 owns A blocks gw * 4 + 0..3 of each half (A1 first, then A0), group
    // 1 owns W blocks gw * 8 + 0..7 (1 KB blocks of 8 staged rows).  Lane l of a block lands at row l / 8, chunk
    // position l % 8 and fetches the logical chunk the swizzle stores there, which depends on the block's parity only.
    // A load's byte offset is the block's first row times K (wave-uniform) plus a per-lane part; rows past M (or N)
    // fall outside the buffer and read as zeros (their results are never stored).
    const __amdgpu_buffer_rsrc_t rs = grp == 0 ? make_rsrc(a, (long)M * K) : make_rsrc(w, (long)N * K);
    const int drow = lane / CPR, pch = lane % CPR;
    const int ch0 = pch ^ swz<CPR>(drow), ch1 = pch ^ swz<CPR>(8 + drow);   // blocks of even / odd index
    const unsigned lane0 = (unsigned)(drow * K + ch0 * 16), lane1 = (unsigned)(drow * K + ch1 * 16);
    const unsigned org = (unsigned)(grp == 0 ? m0 : n0);
    uint8_t* const lbase = reinterpret_cast<uint8_t*>(ldsx);
    // load q of this wavefront for stage `st` into stage buffer st % 2
    auto load = [&](int q, int st) {
        const int blk = grp == 0 ? (q < 4 ? 16 : 0) + gw * 4 + (q & 3) : gw * 8 + q;   // block within A or W
        const int lrow = (grp == 0 ? 0 : BM) + blk * RPB;                                 // staged row in the buffer
        const unsigned base = (org + (unsigned)(blk * RPB)) * (unsigned)K;
        const int k0 = (kst0 + st) * KB;
        unsigned voff = base + ((q & 1) ? lane1 : lane0);
        if constexpr (!KFULL) {                          // a K chunk past the end reads as zeros
            if (k0 + ((q & 1) ? ch1 : ch0) * 16 >= K) voff = 0x7fffffffu;
        }
        dma_block(rs, lbase + (st & 1) * Cfg::STAGE_BYTES + lrow * KB, (int)voff, k0);
    };

    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;
    v4i fa[SUBS][FM], fw[SUBS][FN];
    auto read_frags = [&](int st) {                     // memory phase: every fragment of stage st into registers
        const v4i* la = reinterpret_cast<const v4i*>(lbase + (st & 1) * Cfg::STAGE_BYTES);
        const v4i* lw = la + BM * CPR;
#pragma unroll
        for (int sub = 0; sub < SUBS; ++sub) {
            const int cc = 2 * sub + (lane >> 5);
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int row = grp * WTM + i * 32 + (lane & 31);
                fa[sub][i] = la[row * CPR + (cc ^ swz<CPR>(row))];
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int row = gw * WTN + j * 32 + (lane & 31);
                fw[sub][j] = lw[row * CPR + (cc ^ swz<CPR>(row))];
            }
        }
    };
    // compute phase: the stage's 32 MFMAs, with loads 0..3 (stage st_a) if HA and loads 4..7 (stage st_b) if HB issued
    // one after every 4 MFMAs (HA, HB compile-time, so no branch sits between the MFMAs)
    auto compute = [&](auto HA, auto HB, int st_a, int st_b) {
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int sub = 0; sub < SUBS; ++sub) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int i = 2 * h; i < 2 * h + 2; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fw[sub][j], fa[sub][i], acc[i][j], 0, 0, 0);
                const int q = sub * 2 + h;               // load q: 0..3 of pass a, 4..7 of pass b
                __builtin_amdgcn_sched_barrier(0);
                if (q < 4) {
                    if constexpr (decltype(HA)::value) load(q, st_a);
                } else {
                    if constexpr (decltype(HB)::value) load(q, st_b);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    };
    using Y = std::integral_constant<bool, true>;
    using NO = std::integral_constant<bool, false>;
    auto slot_end = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };
    auto wait_vm = [&](int n) {                         // at most n of this wavefront's loads outstanding
        if (n >= 8) __builtin_amdgcn_s_waitcnt(waitcnt_vm(8));
        else if (n >= 4) __builtin_amdgcn_s_waitcnt(waitcnt_vm(4));
        else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    };
    constexpr int LGKM0 = 0xc07f;

    // prologue: stage 0 whole (group 0: A1 and A0, group 1: W), group 0 also A0 of stage 1, group 1 also W of stage 1
#pragma unroll
    for (int q = 0; q < 8; ++q) load(q, 0);
    if (nk > 1) {
        if (grp == 0) {
#pragma unroll
            for (int q = 4; q < 8; ++q) load(q, 1);
        } else {
#pragma unroll
            for (int q = 0; q < 8; ++q) load(q, 1);
        }
    }
    wait_vm(nk > 1 ? (grp == 0 ? 4 : 8) : 0);            // stage 0 landed
    slot_end();
    // Each stage j: memory phase, then compute phase.  Group 0's compute phase of stage j loads A1 of stage j + 1 and
    // A0 of stage j + 2, group 1's loads W of stage j + 2, where those stages exist; the last two stages are peeled so
    // that which loads exist is known at compile time.
    if (grp == 0) {
        auto stage = [&](int j, auto HA, auto HB) {
            read_frags(j);                              // slot 2j: memory phase
            __builtin_amdgcn_s_waitcnt(LGKM0);
            wait_vm(j + 1 < nk ? 4 : 0);                // A1 of stage j landed (A0 of stage j + 1 may be in flight)
            slot_end();
            compute(HA, HB, j + 1, j + 2);              // slot 2j + 1: MFMAs, A1 of j + 1, A0 of j + 2
            wait_vm(4 * decltype(HA)::value + 4 * decltype(HB)::value);   // A0 of stage j + 1 landed
            slot_end();
        };
        int j = 0;
        for (; j + 2 < nk; ++j) stage(j, Y{}, Y{});
        if (j + 1 < nk) stage(j++, Y{}, NO{});
        stage(j, NO{}, NO{});
    } else {
        auto stage = [&](int j, auto HW, auto LAST) {
            read_frags(j);                              // slot 2j + 1: memory phase
            __builtin_amdgcn_s_waitcnt(LGKM0);
            wait_vm(0);                                 // W of stage j + 1 landed
            slot_end();
            compute(HW, HW, j + 2, j + 2);              // slot 2j + 2: MFMAs, W of stage j + 2
            if constexpr (!decltype(LAST)::value) slot_end();
        };
        slot_end();                                     // slot 0: group 0 reads stage 0
        int j = 0;
        for (; j + 2 < nk; ++j) stage(j, Y{}, NO{});
        if (j + 1 < nk) stage(j++, NO{}, NO{});
        stage(j, NO{}, Y{});
    }
    // Epilogue: group 0 starts while group 1 computes the last stage (slot 2 nk).  Every load has landed and the last
    // reads of the stage buffers ended before the barrier closing slot 2 nk - 1, and each wavefront transposes through
    // its own LDS region, so no further barrier is needed (both groups passed 2 nk + 1).

    // (slots and counters indexed from the first split tile)
    if (split_role && !split_exchange<FM, FN, WM * WN>(acc, ws, rt, piece, splits, wave, lane, tid)) return;

    const int mb = m0 + grp * WTM, nbw = n0 + gw * WTN;
    if constexpr (EPI == EPI_I32) {
        store_tile_i32<FM, FN>(acc, static_cast<int*>(out), M, N, mb, nbw, lane);
    } else {
        store_tile_lds<T, EPI, FM, FN, PITCH>(acc, reinterpret_cast<uint8_t*>(ldsx) + wave * WTM * PITCH, out, sa, sw,
                                              bias, M, N, sa_rows, sw_rows, mb, nbw, lane);
    }
}

// ---------------------------------------------------------------------------------------------------------------------
// stream_lds_kernel: M <= 16 * MT rows, weights streamed once through per-wavefront LDS rings
// ---------------------------------------------------------------------------------------------------------------------
// The MFMA operand layout wants 16 different weight rows in one load instruction, which the vector L1 serves with tag
// conflicts.  Here every load is a direct-to-LDS buffer_load of 1 KB that covers 8 rows x 128 contiguous bytes, and
// the fragments are read from LDS in the MFMA layout.  A workgroup is one 16-row weight tile; its 4 wavefronts take
// interleaved 128-byte K steps, each through its own ring of NS step buffers (16 weight rows, then 16 MT activation
// rows, each 128 bytes with the 8-chunk swizzle), so a wavefront only waits for its own loads and no barrier runs in
// the main loop.  Activation rows past M and K chunks past K are loaded from outside the buffer, which writes zeros.
__device__ __forceinline__ void dma_step(__amdgpu_buffer_rsrc_t rsw, __amdgpu_buffer_rsrc_t rsa, uint8_t* dst,
                                         const int* off, const int* chk, int lps, int k0, int K, int wloads = 2) {
#pragma unroll
    for (int j = 0; j < lps; ++j) {
        const bool ok = k0 + chk[j] * 16 < K;
        if (j < wloads)                                  // weights (the first wloads blocks), read once: non-temporal
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, (lds_void*)(dst + j * 1024), 16, ok ? off[j] : 0x7fffffff,
                                                     k0, 0, CPOL_NT);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_void*)(dst + j * 1024), 16, ok ? off[j] : 0x7fffffff,
                                                     k0, 0, 0);
    }
}

template <typename T, int MT, int NS, int EPI, int KS = 4, int RT = 1>
__global__ void __launch_bounds__(256) stream_lds_kernel(const int8_t* __restrict__ a, const int8_t* __restrict__ w,
                                                         const float* __restrict__ sa, const float* __restrict__ sw,
                                                         const uint16_t* __restrict__ bias, void* __restrict__ out,
                                                         int M, int N, int K, int sa_rows, int sw_rows) {
    constexpr int WR = 16 * RT;                          // weight rows per workgroup (RT tiles of 16)
    constexpr int ROWS = WR + 16 * MT;                   // staged rows per step: weights, then activations
    constexpr int STEP_BYTES = ROWS * 128;
    constexpr int LPS = ROWS / 8;                        // 1 KB loads per step
    extern __shared__ v4i ldsx[];
    // The ring address of every direct-to-LDS load derives from the wavefront index and must be scalar (M0).  With the
    // index from threadIdx the compiler wraps each load in a loop over the index's distinct values (one pass: it is
    // uniform), which also spreads the step's loads through the iteration; in a scalar register the loads go out
    // together.  Same bits either way; measured (same box): the scalar form 48 rows x N 12288 32.05 -> 30.04 us,
    // 64 rows x N 5120 x K 17408 38.2 -> 37.6, but decode M = 6 / 8 / 16 17.91 / 18.42 / 20.74 -> 18.13 / 18.94 /
    // 21.53 us (M = 32 unchanged), so it is taken for MT >= 3 only.
    const int ks = MT >= 3 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int n0 = blockIdx.x * WR;
    uint8_t* const ring = reinterpret_cast<uint8_t*>(ldsx) + ks * NS * STEP_BYTES;
    const __amdgpu_buffer_rsrc_t rsa = make_rsrc(a, (long)M * K), rsw = make_rsrc(w, (long)N * K);
    int off[LPS], chk[LPS];
#pragma unroll
    for (int j = 0; j < LPS; ++j) {
        const int row = j * 8 + (lane >> 3);             // staged row; lane % 8 is the physical chunk
        chk[j] = (lane & 7) ^ swz<8>(row);
        if (j < WR / 8) off[j] = n0 + row < N ? (n0 + row) * K + chk[j] * 16 : 0x7fffffff;
        else off[j] = row - WR < M ? (row - WR) * K + chk[j] * 16 : 0x7fffffff;
    }
    const int nsteps = (K + 127) >> 7;
    const int mine = ks < nsteps ? (nsteps - 1 - ks) / KS + 1 : 0;   // own steps ks, ks + KS, ...
    auto issue = [&](int i) {
        dma_step(rsw, rsa, ring + (i % NS) * STEP_BYTES, off, chk, LPS, (ks + i * KS) * 128, K, WR / 8);
    };
    v4i acc[RT][MT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[rt][mt] = v4i{0, 0, 0, 0};
    const int r = lane & 15, g = lane >> 4;
    auto compute = [&](int slot) {
        const v4i* st = reinterpret_cast<const v4i*>(ring + slot * STEP_BYTES);
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            const int c = 4 * sub + g;                   // this lane's 16-byte chunk of the 128-byte step
            v4i fa[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int ra = WR + 16 * mt + r;
                fa[mt] = st[ra * 8 + (c ^ swz<8>(ra))];
            }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const int rw = rt * 16 + r;
                const v4i fw = st[rw * 8 + (c ^ swz<8>(rw))];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[rt][mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fw, fa[mt], acc[rt][mt], 0, 0, 0);
            }
        }
    };
    constexpr int WAIT2 = waitcnt_vm(2 * LPS), WAIT1 = waitcnt_vm(LPS), WAIT0 = waitcnt_vm(0);
#pragma unroll
    for (int i = 0; i < NS - 1; ++i)
        if (i < mine) issue(i);
    for (int i = 0; i < mine; ++i) {
        // own step i has landed once at most the later steps' loads (LPS each) remain outstanding
        const int ahead = min(mine - 1 - i, NS - 2);
        if (ahead >= 2) __builtin_amdgcn_s_waitcnt(WAIT2);
        else if (ahead == 1) __builtin_amdgcn_s_waitcnt(WAIT1);
        else __builtin_amdgcn_s_waitcnt(WAIT0);
        // the slot of step i - 1, whose fragments this wavefront has already consumed
        if (i + NS - 1 < mine) issue(i + NS - 1);
        compute(i % NS);
    }

    // K slices meet in LDS (after every wavefront is done with its ring)
    __syncthreads();
    int* red = reinterpret_cast<int*>(ldsx) + lane;
    constexpr int PER = RT * MT * 4;                     // partial sums per lane
    if (ks > 0) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int v = 0; v < 4; ++v) red[((ks - 1) * PER + (rt * MT + mt) * 4 + v) * 64] = acc[rt][mt][v];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int q = 0; q < KS - 1; ++q)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[rt][mt][v] += red[(q * PER + (rt * MT + mt) * 4 + v) * 64];
    // D fragment of v_mfma_i32_16x16x64_i8: lane holds rows 4 g + v (weight rows n) of column r (activation row m)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int m = mt * 16 + r;
            if (m >= M) continue;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = n0 + rt * 16 + 4 * g + v;
                if (n < N)
                    store_out<T, EPI>(out, (long)m * N + n, acc[rt][mt][v], sa, sa_rows ? m : 0, sw, sw_rows ? n : 0,
                                      bias);
            }
        }
}

// ---------------------------------------------------------------------------------------------------------------------
// w8a16_kernel: int8 weights (per-row float32 scale) x fp16 / bf16 activations, the int8 LM head, M <= 16 * MT rows
// ---------------------------------------------------------------------------------------------------------------------
// out[m, n] = RN_T( fma( sum_k float(w[n, k]) * float(x[m, k]), s[n], bias[n] or +0 ) )   (csrc/w8a16_gemv.cu:98-117,
// float32 sums; the order of the sum is this kernel's own: the MFMA's and then the 4 K slices in order).
// The weight stream is the LDS-ring design of stream_lds_kernel (RT tiles of 16 weight rows per workgroup, 4
// wavefronts on interleaved 128-byte K steps, direct-to-LDS loads of 8 rows x 128 bytes); each 8-byte weight fragment
// is widened to 8 fp16 / bf16 values in registers and fed to v_mfma_f32_16x16x32_{f16,bf16} as the A operand, the
// activations (read from L2, 16 bytes per lane, once per K step for all RT tiles) as the B operand.  GATHER: weight
// rows rows[n] (a gathered vocabulary subset).
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __bf16 bh8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// 8 int8 -> 8 fp16, exact: byte b becomes the fp16 with bits 0x6400 | (b ^ 0x80), i.e. 1024 + (b + 128), minus 1152.
__device__ __forceinline__ h8 widen_f16(uint32_t lo, uint32_t hi) {
    const uint32_t a = lo ^ 0x80808080u, b = hi ^ 0x80808080u;
    const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const h2 p0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u)) - bias;
    const h2 p1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u)) - bias;
    const h2 p2 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u)) - bias;
    const h2 p3 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u)) - bias;
    return h8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}
// 8 int8 -> 8 bf16, exact: through float32 (|b| <= 128 fits the 8-bit bf16 significand, so the high half is exact).
__device__ __forceinline__ bh8 widen_bf16(uint32_t lo, uint32_t hi) {
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t src = i < 2 ? lo : hi;
        const float f0 = (float)(int8_t)((src >> (16 * (i & 1))) & 0xff);
        const float f1 = (float)(int8_t)((src >> (16 * (i & 1) + 8)) & 0xff);
        o[i] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
    }
    return __builtin_bit_cast(bh8, make_uint4(o[0], o[1], o[2], o[3]));
}

template <typename T, int MT, int NS, bool GATHER, int RT = 1>
__global__ void __launch_bounds__(256) w8a16_kernel(const uint16_t* __restrict__ x, const int8_t* __restrict__ w,
                                                    const float* __restrict__ s, const uint16_t* __restrict__ bias,
                                                    uint16_t* __restrict__ out, int M, int N, int K, int w_rows,
                                                    const int* __restrict__ rows) {
    constexpr int KS = 4, STEP_BYTES = RT * 16 * 128, LPS = 2 * RT;   // RT 16-row tiles share each activation load
    extern __shared__ v4i ldsx[];
    // the wavefront index in a scalar register: the ring address of every direct-to-LDS load derives from it and must be
    // scalar (M0); taken from threadIdx it made the compiler wrap each load in a loop over the index's values (N 248320,
    // K 5120: M = 4 221.5 -> 216.7 us, M = 16 290.2 -> 288.2, same bits)
    const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int n0 = blockIdx.x * 16 * RT;
    uint8_t* const ring = reinterpret_cast<uint8_t*>(ldsx) + ks * NS * STEP_BYTES;
    const __amdgpu_buffer_rsrc_t rsw = make_rsrc(w, (long)w_rows * K);
    int off[LPS], chk[LPS];
#pragma unroll
    for (int j = 0; j < LPS; ++j) {
        const int row = j * 8 + (lane >> 3);
        chk[j] = (lane & 7) ^ swz<8>(row);
        const int n = n0 + row;
        const int src = n < N ? (GATHER ? min(max(rows[n], 0), w_rows - 1) : n) : 0;   // a bad index stays in w
        off[j] = n < N ? src * K + chk[j] * 16 : 0x7fffffff;
    }
    const int nsteps = (K + 127) >> 7;
    const int mine = ks < nsteps ? (nsteps - 1 - ks) / KS + 1 : 0;
    const int r = lane & 15, g = lane >> 4;
    // The step's activation fragments are loaded with its weights, into a register ring beside the LDS ring, from
    // clamped (in-bounds) addresses and masked where used: loaded where used, under the m < M && k < K condition, each
    // was waited for before its MFMA.
    uint4 xr[NS][4][MT];
    auto issue = [&](int i, int slot) {
        const int k0 = (ks + i * KS) * 128;
        dma_step(rsw, rsw, ring + slot * STEP_BYTES, off, chk, LPS, k0, K, LPS);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int m = min(mt * 16 + r, M - 1), k = min(k0 + 32 * j + 8 * g, K - 8);
                xr[slot][j][mt] = *reinterpret_cast<const uint4*>(x + (long)m * K + k);
            }
    };
    f4 acc[RT][MT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[rt][mt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](int slot, int k0) {
        const uint8_t* st = ring + slot * STEP_BYTES;
#pragma unroll
        for (int j = 0; j < 4; ++j) {                    // 32-element MFMA K blocks of the 128-byte step
            const int c = 2 * j + (g >> 1);
            const int k = k0 + 32 * j + 8 * g;           // this lane's 8 activations
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const int wr = rt * 16 + r;              // staged weight row
                const uint2 wv = *reinterpret_cast<const uint2*>(st + wr * 128 + (c ^ swz<8>(wr)) * 16 + 8 * (g & 1));
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int m = mt * 16 + r;
                    const uint4 xv = m < M && k < K ? xr[slot][j][mt] : make_uint4(0, 0, 0, 0);
                    if constexpr (__is_same(T, f16))
                        acc[rt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            widen_f16(wv.x, wv.y), __builtin_bit_cast(h8, xv), acc[rt][mt], 0, 0, 0);
                    else
                        acc[rt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            widen_bf16(wv.x, wv.y), __builtin_bit_cast(bh8, xv), acc[rt][mt], 0, 0, 0);
                }
            }
        }
    };
    constexpr int VPS = LPS + 4 * MT;                    // vector memory instructions per step
    constexpr int WAIT2 = waitcnt_vm(2 * VPS), WAIT1 = waitcnt_vm(VPS), WAIT0 = waitcnt_vm(0);
    static_assert(NS == 3, "the register ring is unrolled for three steps");
#pragma unroll
    for (int i = 0; i < NS - 1; ++i)
        if (i < mine) issue(i, i);
    for (int i0 = 0; i0 < mine; i0 += NS) {
#pragma unroll
        for (int u = 0; u < NS; ++u) {                   // step i in slot u (i0 is a multiple of NS)
            const int i = i0 + u;
            if (i >= mine) break;
            const int ahead = min(mine - 1 - i, NS - 2);
            if (ahead >= 2) __builtin_amdgcn_s_waitcnt(WAIT2);
            else if (ahead == 1) __builtin_amdgcn_s_waitcnt(WAIT1);
            else __builtin_amdgcn_s_waitcnt(WAIT0);
            if (i + NS - 1 < mine) issue(i + NS - 1, (u + NS - 1) % NS);
            compute(u, (ks + i * KS) * 128);
        }
    }
    // K slices meet in LDS, in slice order
    __syncthreads();
    float* red = reinterpret_cast<float*>(ldsx) + lane;
    constexpr int PER = RT * MT * 4;                     // partial sums per lane
    if (ks > 0) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    red[((ks - 1) * PER + (rt * MT + mt) * 4 + v) * 64] = acc[rt][mt][v];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int q = 0; q < KS - 1; ++q)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[rt][mt][v] += red[(q * PER + (rt * MT + mt) * 4 + v) * 64];
    // D of v_mfma_f32_16x16x32: lane holds rows 4 g + v (weight rows) of column r (activation row)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int m = mt * 16 + r;
            if (m >= M) continue;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int n = n0 + rt * 16 + 4 * g + v;
                if (n >= N) continue;
                const int src = GATHER ? min(max(rows[n], 0), w_rows - 1) : n;
                const float b = bias ? to_float(T{bias[src]}) : 0.0f;
                out[(long)m * N + n] = from_float<T>(__builtin_fmaf(acc[rt][mt][v], s[src], b));
            }
        }
}

// w8a16_dot_kernel: M <= 2 rows of the int8 LM head through the VALU.  The weight stream of gemv_dot4_kernel (each
// wavefront instruction reads 1 KB of one weight row, non-temporally; lane l owns the 16-byte chunks l, l + 64, ...;
// rows grid-strided over at most four resident workgroups per CU, the next row's loads issued before this row's math);
// each lane widens its 16 weights to 16-bit pairs (fp16 by the exact bit trick, bf16 through float32) and
// accumulates v_dot2_f32_{f16,bf16} against the activations it keeps in registers; a row's float32 partial sums meet
// across the wavefront (DPP, ds_swizzle, readlane; every lane ends with the same sum).  Sum order: each lane's chain
// over its chunks, then the wavefront tree.
typedef __bf16 bh2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float wave_sum_f(float v) {
    v += dpp_f<0xB1>(v);                               // lane ^ 1
    v += dpp_f<0x4E>(v);                               // lane ^ 2
    v += dpp_f<0x141>(v);                              // row_half_mirror: groups of 8
    v += dpp_f<0x140>(v);                              // row_mirror: rows of 16
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));   // lane ^ 16
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
}

// one dword of 4 int8 weights -> the 16-bit pairs (elements 0, 1) and (2, 3), exactly
__device__ __forceinline__ void widen4(uint32_t d, uint32_t& p0, uint32_t& p1, f16) {
    const uint32_t a = d ^ 0x80808080u;
    const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const h2 lo = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, a, 0x04010400u));
    const h2 hi = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u));
    p0 = __builtin_bit_cast(uint32_t, lo - bias);
    p1 = __builtin_bit_cast(uint32_t, hi - bias);
}
__device__ __forceinline__ void widen4(uint32_t d, uint32_t& p0, uint32_t& p1, bf16) {
    const float f0 = (float)(int8_t)(d & 0xff), f1 = (float)(int8_t)((d >> 8) & 0xff);
    const float f2 = (float)(int8_t)((d >> 16) & 0xff), f3 = (float)(int8_t)(d >> 24);
    p0 = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
    p1 = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
}
__device__ __forceinline__ float dot2(uint32_t w2, uint32_t x2, float acc, f16) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, w2), __builtin_bit_cast(h2, x2), acc, false);
}
__device__ __forceinline__ float dot2(uint32_t w2, uint32_t x2, float acc, bf16) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bh2, w2), __builtin_bit_cast(bh2, x2), acc, false);
}

template <typename T, int M, int CH, bool GATHER>
__global__ void __launch_bounds__(256) w8a16_dot_kernel(const uint16_t* __restrict__ x, const int8_t* __restrict__ w,
                                                        const float* __restrict__ s, const uint16_t* __restrict__ bias,
                                                        uint16_t* __restrict__ out, int N, int K, int w_rows,
                                                        const int* __restrict__ rows) {
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * (blockDim.x >> 6);
    const int wid = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int K16 = K >> 4;
    const v4i z = {0, 0, 0, 0};
    v4i xv[M][CH][2];                                    // 16 activations (32 bytes) per chunk and row
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int c = lane + 64 * j;
            const v4i* src = reinterpret_cast<const v4i*>(x + (long)m * K + c * 16);
            xv[m][j][0] = c < K16 ? src[0] : z;
            xv[m][j][1] = c < K16 ? src[1] : z;
        }
    auto src_row = [&](int n) { return GATHER ? min(max(rows[n], 0), w_rows - 1) : n; };
    v4i wb[2][CH];
    float sb[2];                                         // the row's scale and bias bits, loaded with the row
    uint16_t bb[2];
    auto load = [&](int buf, int n) {
        const int sr = src_row(n);
        const int8_t* row = w + (long)sr * K;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int c = lane + 64 * j;
            wb[buf][j] = wload<true>(row + min(c, K16 - 1) * 16);   // unmasked (see gemv_dot4_kernel)
        }
        sb[buf] = s[sr];
        bb[buf] = gload<uint16_t>(bias ? bias + sr : &g_zero16);   // unconditional (see gemv_dot4_kernel)
    };
    auto finish = [&](int buf, int n) {
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {              // weight dword e: elements 4 e .. 4 e + 3 of the chunk
                uint32_t p0, p1;
                widen4((uint32_t)wb[buf][j][e], p0, p1, T{});
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    acc[m] = dot2(p0, (uint32_t)xv[m][j][e >> 1][2 * (e & 1)], acc[m], T{});
                    acc[m] = dot2(p1, (uint32_t)xv[m][j][e >> 1][2 * (e & 1) + 1], acc[m], T{});
                }
            }
            // one chunk at a time: left free, the scheduler widens every chunk up front (bf16: 156 registers)
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float t = wave_sum_f(acc[m]);
            if (lane == m) out[(long)m * N + n] = from_float<T>(__builtin_fmaf(t, sb[buf], to_float(T{bb[buf]})));
        }
    };
    // rows wid, wid + nw, ...: peeled as in gemv_dot4_kernel so that no load sits under a condition
    if (wid >= N) return;
    const int cnt = (N - 1 - wid) / nw + 1;
    load(0, wid);
    int k = 0;
    for (; k + 2 < cnt; k += 2) {
        load(1, wid + (k + 1) * nw);
        finish(0, wid + k * nw);
        load(0, wid + (k + 2) * nw);
        finish(1, wid + (k + 1) * nw);
    }
    if (k + 1 < cnt) {
        load(1, wid + (k + 1) * nw);
        finish(0, wid + k * nw);
        finish(1, wid + (k + 1) * nw);
    } else {
        finish(0, wid + k * nw);
    }
}

// ---------------------------------------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------------------------------------

struct Args {
    const int8_t* a;
    const int8_t* w;
    const float* sa;
    const float* sw;
    const uint16_t* bias;
    void* out;
    int M, N, K, sa_rows, sw_rows;
    hipStream_t st;
    // the VALU GEMV with in-kernel activation quantization: 16-bit rows x (stride ldx), int8 copy xq, scales xs
    const uint16_t* x = nullptr;
    long ldx = 0;
    int8_t* xq = nullptr;
    float* xs = nullptr;
    // the prefill GEMM's K-split remainder: a workspace of tile counters (zero between calls) and accumulator slots
    int* ws = nullptr;
    long ws_bytes = 0;
};

// One to five activation rows: the VALU kernel (measured against the LDS-ring MFMA kernel with ordinary loads: 16.8
// vs 18.1 us at K = 5120, N = 17408), at one row up to K = 17408 (17.5 vs 19.4 us at N = 5120), at two or three rows
// up to K = 8192 (past that the LDS-ring kernel won, 19.6 vs 22.0 us at K = 17408, M = 2), at four or five rows up
// to K = 5120.  At K = 5120, N = 17408: M=3 16.2 vs 18.4 us, M=4 17.0 vs 18.4, M=5 17.7 vs 18.6; six rows tie and
// seven or eight lose (19.2 / 21.2 / 21.6 vs 19.0 / 19.1 / 19.5 us: the activations' registers cut occupancy).
// Chunk counts are rounded up to the next of 1..8, 10, 12, 14, 17 (chunks past K are masked).
constexpr int DOT4_MAX_M = 5, DOT4_MAX_CH = 17, DOT4_MAX_CH_M2 = 8, DOT4_MAX_CH_M4 = 5;

static int dot4_chunks(int K) {
    const int c = (K / 16 + 63) / 64;
    return c <= 8 ? c : c <= 10 ? 10 : c <= 12 ? 12 : c <= 14 ? 14 : c <= 17 ? 17 : 1 << 20;
}

// Grid for M >= 3: at most DOT4_BLOCKS_PER_CU workgroups per CU that are resident together (fewer when the registers
// of a long K allow fewer), the same number on every CU, rows grid-strided over their wavefronts.  At K = 5120,
// N = 17408 with non-temporal weight loads: M=1 16.9 -> 15.1 us, M=2 19.3 -> 15.8 us against one wavefront per two
// rows with ordinary loads (the non-temporal loads alone: 15.1 and 17.6 us).
constexpr int DOT4_BLOCKS_PER_CU = 4;
// M <= 2 instead: one wavefront per workgroup and ceil(N / DOT4_ROWS_PER_WAVE) of them, so that every wavefront has
// the same number of rows (four workgroups of four wavefronts per CU leave 4.25 rows per wavefront at N = 17408, a
// last quarter-round with a quarter of the wavefronts).  Against that grid, two runs at K = 5120: N = 17408 M=1
// 14.93-14.98 -> 14.73-14.77 us, M=2 15.57 -> 15.40 us; N = 34816 M=1 27.8 -> 27.2 us, M=2 28.4 -> 27.4 us; and
// N = 5120, K = 17408, M=1 15.7 -> 15.5 us.  Two or four rows per wavefront: as fast at M = 1, K = 5120, up to 6%
// slower elsewhere; at M = 3 the registers allow fewer wavefronts and this grid is 13% slower.
constexpr int DOT4_ROWS_PER_WAVE = 3;

// Workgroups per CU of a row-streaming VALU kernel (256 threads, no LDS): DOT4_BLOCKS_PER_CU, or as many as are
// resident together if fewer (its caller keeps the answer in a static per kernel).
static int row_stream_per_cu(const void* kern) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, 256, 0) != hipSuccess || nb < 1) nb = 1;
    return nb < DOT4_BLOCKS_PER_CU ? nb : DOT4_BLOCKS_PER_CU;
}

template <typename T, int M, int CH, int EPI, bool QX = false>
static void launch_dot4_ch(const Args& p) {
    if constexpr (CH <= DOT4_MAX_CH && (M < 2 || CH <= DOT4_MAX_CH_M2) && (M < 4 || CH <= DOT4_MAX_CH_M4)) {
        using K_ = decltype(&gemv_dot4_kernel<T, M, CH, 1, EPI, true, QX>);
        const K_ kern = &gemv_dot4_kernel<T, M, CH, 1, EPI, true, QX>;
        if constexpr (QX) {                              // 4-wavefront workgroups sharing the quantized rows in LDS
            const int lds = M * CH * 1024 + 64;          // rows of up to CH * 1024 int8, then the reduction floats
            static const int per_cu = [&] {
                int nb = 0;
                if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, reinterpret_cast<const void*>(kern), QX_THREADS,
                                                                 lds) != hipSuccess || nb < 1)
                    nb = 1;
                return nb < DOT4_BLOCKS_PER_CU ? nb : DOT4_BLOCKS_PER_CU;
            }();
            // three rows per wavefront, as the plain kernel's one-row grid: every workgroup quantizes the row again,
            // so fewer, fuller workgroups (one row per wavefront: K = 6144, N = 5120 9.07 -> 8.55 us; K = 17408
            // 18.83 -> 18.62 us; two rows per wavefront no better)
            const int need = (p.N + 11) / 12, grid = cu_count() * per_cu;
            kern<<<need < grid ? need : grid, QX_THREADS, p.M * p.K + 64, p.st>>>(
                p.a, p.w, p.sa, p.sw, p.bias, p.out, p.N, p.K, p.sa_rows, p.sw_rows, p.x, p.ldx, p.xq, p.xs);
            return;
        }
        if constexpr (M <= 2) {                          // every wavefront DOT4_ROWS_PER_WAVE rows: stores deferred
            static_assert(DOT4_ROWS_PER_WAVE == 3, "the deferred-store kernel takes three row groups");
            const int waves = (p.N + DOT4_ROWS_PER_WAVE - 1) / DOT4_ROWS_PER_WAVE;
            gemv_dot4_kernel<T, M, CH, 1, EPI, true, false, false, 3><<<waves, 64, 0, p.st>>>(
                p.a, p.w, p.sa, p.sw, p.bias, p.out, p.N, p.K, p.sa_rows, p.sw_rows, p.x, p.ldx, p.xq, p.xs);
            return;
        }
        static const int per_cu = row_stream_per_cu(reinterpret_cast<const void*>(kern));
        const int need = (p.N + 3) / 4, grid = cu_count() * per_cu;
        kern<<<need < grid ? need : grid, 256, 0, p.st>>>(p.a, p.w, p.sa, p.sw, p.bias, p.out, p.N, p.K, p.sa_rows,
                                                          p.sw_rows, p.x, p.ldx, p.xq, p.xs);
    }
}
template <typename T, int M, int EPI, bool QX = false>
static void launch_dot4_m(const Args& p) {
    if constexpr (M <= DOT4_MAX_M) {
        switch (dot4_chunks(p.K)) {
#define W8_CASE(C) case C: launch_dot4_ch<T, M, C, EPI, QX>(p); break;
            W8_CASE(1) W8_CASE(2) W8_CASE(3) W8_CASE(4) W8_CASE(5) W8_CASE(6) W8_CASE(7) W8_CASE(8) W8_CASE(10)
            W8_CASE(12) W8_CASE(14) W8_CASE(17)
#undef W8_CASE
        }
    }
}
// gate_up with SiLU * up (SILU above): p.N pairs; at M <= 2 one wavefront per workgroup with two pairs (four rows)
// each, else the grid of the plain kernel.
template <typename T, int M, int CH>
static void launch_dot4_silu_ch(const Args& p) {
    if constexpr (CH <= DOT4_MAX_CH && (M < 2 || CH <= DOT4_MAX_CH_M2) && (M < 4 || CH <= DOT4_MAX_CH_M4)) {
        const auto kern = &gemv_dot4_kernel<T, M, CH, 2, EPI_SMALL, true, false, true>;
        if constexpr (M <= 2) {
            kern<<<(p.N + 1) / 2, 64, 0, p.st>>>(p.a, p.w, p.sa, p.sw, p.bias, p.out, p.N, p.K, p.sa_rows, p.sw_rows,
                                                 nullptr, 0, nullptr, nullptr);
            return;
        }
        static const int per_cu = row_stream_per_cu(reinterpret_cast<const void*>(kern));
        const int need = (p.N + 3) / 4, grid = cu_count() * per_cu;
        kern<<<need < grid ? need : grid, 256, 0, p.st>>>(p.a, p.w, p.sa, p.sw, p.bias, p.out, p.N, p.K, p.sa_rows,
                                                          p.sw_rows, nullptr, 0, nullptr, nullptr);
    }
}
template <typename T, int M>
static void launch_dot4_silu_m(const Args& p) {
    switch (dot4_chunks(p.K)) {
#define W8_CASE(C) case C: launch_dot4_silu_ch<T, M, C>(p); break;
        W8_CASE(1) W8_CASE(2) W8_CASE(3) W8_CASE(4) W8_CASE(5) W8_CASE(6) W8_CASE(7) W8_CASE(8) W8_CASE(10)
        W8_CASE(12) W8_CASE(14) W8_CASE(17)
#undef W8_CASE
    }
}
template <typename T>
static void launch_dot4_silu(const Args& p) {
    switch (p.M) {
        case 1: launch_dot4_silu_m<T, 1>(p); break;
        case 2: launch_dot4_silu_m<T, 2>(p); break;
        case 3: launch_dot4_silu_m<T, 3>(p); break;
        case 4: launch_dot4_silu_m<T, 4>(p); break;
        case 5: launch_dot4_silu_m<T, 5>(p); break;
    }
}

static bool dot4_ok(const Args& p) {
    return p.M <= DOT4_MAX_M &&
           dot4_chunks(p.K) <= (p.M < 2 ? DOT4_MAX_CH : p.M < 4 ? DOT4_MAX_CH_M2 : DOT4_MAX_CH_M4);
}

template <typename T, int EPI, bool QX = false>
static void launch_dot4(const Args& p) {
    switch (p.M) {
        case 1: launch_dot4_m<T, 1, EPI, QX>(p); break;
        case 2: launch_dot4_m<T, 2, EPI, QX>(p); break;
        case 3: launch_dot4_m<T, 3, EPI, QX>(p); break;
        case 4: launch_dot4_m<T, 4, EPI, QX>(p); break;
        case 5: launch_dot4_m<T, 5, EPI, QX>(p); break;
    }
}

// M <= 32 past the VALU kernel: the MFMA kernel through per-wavefront LDS rings of 3 steps (48 or 72 KB per
// workgroup: three or two workgroups per CU); measured against 2 and 4 steps, and against loads straight into
// registers (the LDS rings take M = 8, K = 5120, N = 17408 from 23.6 to 18.9 us and M = 32 from 45.6 to 28.1 us).
// One workgroup per 16-row tile: where the tiles need more than one round of the resident workgroups and the last
// round would be less than half full (a quarter-full last round ran at ~40% of the bandwidth: at M = 8, N = 13312
// took 16.9 us against 12.6 us at N = 12288), a workgroup of two wavefronts (K in two slices) with a 3-step ring, or
// else a 2-step ring, is used if that fits every tile in one round: K = 5120, N = 17408, M = 8 19.6 -> 18.4 us,
// M = 16 21.9 -> 20.9 us, M = 32 30.9 -> 27.4 us.  Where four wavefronts already fill their rounds the narrower
// workgroups are slower (N = 5120, K = 17408, M = 8: 20.4 -> 29.1 us).
template <typename T, int MT, int NS, int KS, int EPI, int RT>
struct SldsCfg {
    static constexpr int LDS = KS * NS * (16 * RT + 16 * MT) * 128;
    static_assert(LDS <= 160 * 1024 && LDS >= (KS - 1) * RT * MT * 4 * 64 * 4, "LDS ring size");
    static const void* kern() { return reinterpret_cast<const void*>(&stream_lds_kernel<T, MT, NS, EPI, KS, RT>); }
    static int slots() {                                 // resident workgroups on the whole GPU
        static const int n = [] {
            (void)hipFuncSetAttribute(kern(), hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
            int nb = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern(), 64 * KS, LDS) != hipSuccess || nb < 1) nb = 1;
            return nb * cu_count();
        }();
        return n;
    }
    static void launch(const Args& p) {
        static const hipError_t attr = hipFuncSetAttribute(kern(), hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
        (void)attr;
        stream_lds_kernel<T, MT, NS, EPI, KS, RT><<<(p.N + 16 * RT - 1) / (16 * RT), 64 * KS, LDS, p.st>>>(
            p.a, p.w, p.sa, p.sw, p.bias, p.out, p.M, p.N, p.K, p.sa_rows, p.sw_rows);
    }
};
// The configuration of RT tiles per workgroup that the round rule picks, launched if `launch`; returns the fraction
// of the resident slot-rounds its workgroups fill.
template <typename T, int MT, int RT, int EPI>
static double stream_lds_plan(const Args& p, bool launch) {
    using Wide = SldsCfg<T, MT, 3, 4, EPI, RT>;
    using Two = SldsCfg<T, MT, 3, 2, EPI, RT>;
    using TwoShort = SldsCfg<T, MT, 2, 2, EPI, RT>;
    const int tiles = (p.N + 16 * RT - 1) / (16 * RT), s0 = Wide::slots(), last = tiles % s0;
    int which = 0, slots = s0;
    if (tiles > s0 && last > 0 && 2 * last < s0) {
        if (tiles <= Two::slots()) which = 1, slots = Two::slots();
        else if (tiles <= TwoShort::slots()) which = 2, slots = TwoShort::slots();
    }
    if (launch) {
        if (which == 1) Two::launch(p);
        else if (which == 2) TwoShort::launch(p);
        else Wide::launch(p);
    }
    const int rounds = (tiles + slots - 1) / slots;
    return (double)tiles / ((double)rounds * slots);
}
// Above 16 rows the activations are 4 KB per 128-byte K step against 2 KB of weights per 16-row tile, so a workgroup
// covers up to three tiles that share each activation fragment: of three, two and one tiles per workgroup the launch
// takes the one whose workgroups fill the most of their slot-rounds (ties to more tiles).  M = 32, K = 5120 against
// one tile: N = 12288 23.8 -> 17.1 us (three), N = 34816 55.5 -> 46.3 (three), N = 6144 13.2 -> 11.8 (two); N = 5120,
// K = 17408 34.0 -> 27.0 us (two; three leave 107 workgroups on 256 CUs).  At M <= 16 (2 KB of activations per
// step) several tiles per workgroup measured slower.
template <typename T, int MT, int EPI>
static void launch_stream_lds(const Args& p) {
    if constexpr (MT == 1) {
        stream_lds_plan<T, 1, 1, EPI>(p, true);
    } else if constexpr (MT == 2) {
        const double f3 = stream_lds_plan<T, MT, 3, EPI>(p, false), f2 = stream_lds_plan<T, MT, 2, EPI>(p, false),
                     f1 = stream_lds_plan<T, MT, 1, EPI>(p, false);
        if (f3 >= f2 && f3 >= f1) stream_lds_plan<T, MT, 3, EPI>(p, true);
        else if (f2 >= f1) stream_lds_plan<T, MT, 2, EPI>(p, true);
        else stream_lds_plan<T, MT, 1, EPI>(p, true);
    } else {                                             // 64 activation rows: three tiles' rings would not fit
        const double f2 = stream_lds_plan<T, MT, 2, EPI>(p, false), f1 = stream_lds_plan<T, MT, 1, EPI>(p, false);
        if (f2 >= f1) stream_lds_plan<T, MT, 2, EPI>(p, true);
        else stream_lds_plan<T, MT, 1, EPI>(p, true);
    }
}

// M <= 32: the VALU kernel where it applies, else the LDS-ring MFMA streaming kernel.
template <typename T, int EPI>
static void launch_stream(const Args& p) {
    if (dot4_ok(p)) launch_dot4<T, EPI>(p);
    else if (p.M <= 16) launch_stream_lds<T, 1, EPI>(p);
    else launch_stream_lds<T, 2, EPI>(p);
}

// Main configuration: 256 x 256 tiles, 2 x 4 wavefronts of 128 x 64, 128-byte K stages, 2 in LDS (128 KB): measured
// ~9% faster than 64-byte stages x 4 at every prefill shape (half the barriers outweigh the shorter prefetch distance),
// and 4-10% faster with the weights read from HBM too (M = 4096, N = 12288: 231 against 245 us).
// Small configuration: 128 x 128 quarter tiles, 2 x 2 wavefronts of 64 x 64, the same stages (64 KB: two workgroups
// per CU).
// Where the next stage's loads are issued (SPLIT slices; LEAD: the first at the barrier): the main configuration issues
// its two slices after the MFMAs of sub-steps 0 and 1 rather than in one burst after the barrier, where the issue
// blocked each wavefront for ~940 of the ~3300 cycles of a stage (s_memtime stamps at M = N = 4096: 253 -> 229 us at
// M 4096 x N 12288 x K 5120).  Long grids (at least LONG_ROUNDS rounds of super tiles over the CUs) measured best
// with the first slice at the barrier (720 -> 695 us at N = 34816; 741 us with the main placement); the small
// configuration best with one burst.
struct MainCfg {
    static constexpr int WM = 2, WN = 4, FM = 4, FN = 2, KB = 128, NS = 2, SPLIT = 2;
    static constexpr bool LEAD = false;
};
struct LongCfg {
    static constexpr int WM = 2, WN = 4, FM = 4, FN = 2, KB = 128, NS = 2, SPLIT = 2;
    static constexpr bool LEAD = true;
};
struct SmallCfg {
    static constexpr int WM = 2, WN = 2, FM = 2, FN = 2, KB = 128, NS = 2, SPLIT = 0;
    static constexpr bool LEAD = false;
};
// The quarter tiles with 4 K stages in LDS (128 KB, one workgroup per CU), for a remainder whose quarter tiles fit in
// one round at one per CU: each workgroup keeps three stages of its rows in flight, which a few workgroups streaming
// long K from HBM need.  Weights rotated beyond the MALL: N = 5120, K = 17408, M = 512 122.3 -> 86.0 us; N = 5120,
// K = 5120, M = 512 43.1 -> 30.6 us; M = 512, N = 34816 (16 remaining super tiles) 126.5 -> 120.7 us against 64 x 128
// eighth tiles with 2 stages, which it replaces; 3 stages measured within 2% of 4.
struct SmallDeepCfg {
    static constexpr int WM = 2, WN = 2, FM = 2, FN = 2, KB = 128, NS = 4, SPLIT = 0;
    static constexpr bool LEAD = false;
};
// Mid configurations for 33..128 rows, where a tile row holds all of M: 64-row tiles with 4 K stages in LDS, so that
// each workgroup has three stages of its weight rows in flight instead of one.  Up to N = 12288: 64 x 128 tiles (96
// KB, one workgroup per CU): K = 5120, N = 12288, M = 96 47.7 -> 25.7 us, M = 128 49.4 -> 27.5; N = 10240, M = 128
// 49.1 -> 26.8 us.  Above: 64 x 64 tiles (2 x 2 wavefronts of 32 x 32, 64 KB, two workgroups per CU), twice as many
// workgroups on the weight stream: N = 17408, M = 33 44.1 -> 29.2 us, M = 64 49.1 -> 34.4, M = 128 47.9 -> 42.1;
// N = 24576, M = 64 53.0 -> 36.5; N = 34816, M = 48 70.7 -> 48.7, M = 128 74.6 -> 70.2 us (at N = 12288, M = 128 the
// 64 x 64 tiles take 30.5 us against 26.8).  Three stages gained less, six no more.  The 64 x 128 tiles also serve
// 129..256 rows against at most 8192 weight rows, where the other configurations have few tiles to spread: N = 5120,
// K = 17408, M = 256 111.8 -> 64.4 us; N = 6144, K = 5120, M = 256 37.0 -> 24.4 us (from N = 12288 on they lose).
struct MidCfg {
    static constexpr int WM = 2, WN = 2, FM = 1, FN = 2, KB = 128, NS = 4, SPLIT = 0;
    static constexpr bool LEAD = false;
};
struct Mid64Cfg {
    static constexpr int WM = 2, WN = 2, FM = 1, FN = 1, KB = 128, NS = 4, SPLIT = 0;
    static constexpr bool LEAD = false;
};
constexpr int MID_GEMM_MAX_M = 128, MID_GEMM_WIDE_N = 12288;
constexpr int LONG_ROUNDS = 6;

// Which configuration covers which super tiles: 0 = main only, 2 = small only, 1 = main for the whole rounds of super
// tiles over the CUs and small for a last partial round of at most CUs / W8_SMALL_REM_DIV super tiles.
#ifndef W8_GEMM_POLICY
#define W8_GEMM_POLICY 1
#endif
#ifndef W8_SMALL_REM_DIV
#define W8_SMALL_REM_DIV 2
#endif

#ifndef W8_GEMM_PP
#define W8_GEMM_PP 1
#endif
// The main configuration with its wavefront groups in alternating roles (gemm_pp_kernel).
template <typename T, int EPI, bool KFULL, bool SPLITK>
static void launch_gemm_pp_k(const Args& p, int t_base, int blocks, int splits, int full) {
    using G = GemmCfg<MainCfg::WM, MainCfg::WN, MainCfg::FM, MainCfg::FN, MainCfg::KB, MainCfg::NS>;
    const void* kern = reinterpret_cast<const void*>(&gemm_pp_kernel<T, EPI, KFULL, SPLITK>);
    static const hipError_t attr = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS_BYTES);
    (void)attr;
    gemm_pp_kernel<T, EPI, KFULL, SPLITK><<<blocks, G::THREADS, G::LDS_BYTES, p.st>>>(
        p.a, p.w, p.sa, p.sw, p.bias, p.out, p.M, p.N, p.K, p.sa_rows, p.sw_rows, t_base, splits, full, p.ws);
}
template <typename T, int EPI>
static void launch_gemm_pp(const Args& p, int t_base, int blocks) {
    if (p.K % MainCfg::KB == 0) launch_gemm_pp_k<T, EPI, true, false>(p, t_base, blocks, 1, 0);
    else launch_gemm_pp_k<T, EPI, false, false>(p, t_base, blocks, 1, 0);
}
// `full` whole tiles from t_base, then `rem` tiles as `splits` K pieces each, in one launch
template <typename T, int EPI>
static void launch_gemm_pp_split(const Args& p, int t_base, int full, int rem, int splits) {
    const int blocks = full + rem * splits;
    if (p.K % MainCfg::KB == 0) launch_gemm_pp_k<T, EPI, true, true>(p, t_base, blocks, splits, full);
    else launch_gemm_pp_k<T, EPI, false, true>(p, t_base, blocks, splits, full);
}

template <typename T, int EPI, typename C, bool KS = false>
static void launch_gemm_cfg(const Args& p, int t_base, int blocks, int splits = 1) {
    using G = GemmCfg<C::WM, C::WN, C::FM, C::FN, C::KB, C::NS>;
    const void* kern = reinterpret_cast<const void*>(
        &gemm_kernel<T, EPI, C::WM, C::WN, C::FM, C::FN, C::KB, C::NS, C::SPLIT, C::LEAD, GROUP_M, false, KS>);
    static const hipError_t attr = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS_BYTES);
    (void)attr;
    gemm_kernel<T, EPI, C::WM, C::WN, C::FM, C::FN, C::KB, C::NS, C::SPLIT, C::LEAD, GROUP_M, false, KS>
        <<<blocks, G::THREADS, G::LDS_BYTES, p.st>>>(
        p.a, p.w, p.sa, p.sw, p.bias, p.out, p.M, p.N, p.K, p.sa_rows, p.sw_rows, t_base, splits, p.ws);
}


// Up to 64 rows against at most 12288 weight rows, or up to 128 rows against at most 8192: the prefill kernel has
// few tiles to spread there (N = 5120: 20 super tiles in a single tile row), so the streaming kernel runs instead, in
// passes of at most 64 rows, with the same epilogue (bit-identical).  Rotated weights, bf16, against the prefill
// kernel: N = 5120, K = 17408, M = 33..64 114 -> 35-38 us, M = 96 113 -> 65 us, M = 128 114 -> 76 us; N = 12288,
// K = 5120, M = 33..64 42-45 -> 31-35 us; N = 8192, M = 128 38 -> 36 us.  Past these bounds the prefill kernel is
// faster (N = 12288, M = 128: 50 against 69 us; N = 17408, M = 33: 46 against 51 us): the passes re-read the weights
// and the 64-row rings leave few wavefronts per CU.  With a workspace the 64 x 64 tiles split over K take most of
// these shapes (mid_split_plan).
static bool mid_stream(int M, int N) { return (M <= 64 && N <= 12288) || (M <= 128 && N <= 8192); }
template <typename T, int EPI>
static void launch_stream_rows(const Args& p) {
    const int esz = EPI == EPI_I32 ? 4 : 2;              // output element bytes
    for (int m0 = 0; m0 < p.M; m0 += 64) {
        Args q = p;
        q.M = min(64, p.M - m0);
        q.a = p.a + (long)m0 * p.K;
        q.out = static_cast<uint8_t*>(p.out) + (long)m0 * p.N * esz;
        if (p.sa_rows) q.sa = p.sa + m0;
        if (q.M <= 16) launch_stream_lds<T, 1, EPI>(q);
        else if (q.M <= 32) launch_stream_lds<T, 2, EPI>(q);
        else launch_stream_lds<T, 4, EPI>(q);
    }
}

// The K-split remainder.  After the whole rounds of super tiles over the CUs, a last partial round of rem <= CUs / 2
// tiles leaves most CUs idle or, as quarter tiles, runs at a lower MFMA rate; instead each of those tiles runs as
// `splits` K pieces on the main configuration (rem * splits <= CUs workgroups), pieces of at least SPLIT_MIN_STAGES
// 128-byte stages, their int32 partial sums met in a workspace.  Same box, rotated weights, against the quarter
// tiles: M 512 x N 12288 x K 5120 (96 x 2) 55.3 -> 44.8 us, M 1024 x N 5120 x K 17408 (80 x 3) 123.8 -> 93.1 us,
// M 4096 x N 5120 x K 17408 (256 whole + 64 x 4) 313.8 -> 299.4 us.  Returns the splits for M x N x K under the
// default policy (1: no split) and the workspace bytes it needs.
// Pieces of at least 16 stages: shorter ones are dominated by a piece's fixed cost (prologue, partial exchange,
// epilogue: ~15 us against ~1.45 us per stage) and lose to, or tie with, the 4-stage quarter tiles (same box: M 512
// x N 34816 x K 5120, 256 whole + 16 tiles as 16 x 8 pieces of 5 stages 111.0 us against 104.9, as 16 x 4 of 10
// stages 103.7 against 105.0; M 4096 x N 17152 x K 5120, 48 x 4 of 10 stages 323.7 against 310.2).
constexpr int SPLIT_MIN_STAGES = 16, SPLIT_MAX = 8;
static bool gemm_mid_path(int M, int N) {
    return mid_stream(M, N) || M <= MID_GEMM_MAX_M || (M <= 2 * MID_GEMM_MAX_M && N <= 8192);
}
static int split_plan(int M, int N, int K, int cus, int* full, int* rem, long* bytes) {
    const int tiles = ((M + SUPER - 1) / SUPER) * ((N + SUPER - 1) / SUPER);
    *full = tiles / cus * cus;
    *rem = tiles - *full;
    *bytes = 0;
    if (gemm_mid_path(M, N) || *rem == 0 || *rem > cus / 2 || *rem > SPLIT_HEAD_INTS) return 1;
    const int nk = (K + 127) / 128;
    const int s = min(min(cus / *rem, nk / SPLIT_MIN_STAGES), SPLIT_MAX);
    // two pieces after whole rounds lose to the quarter tiles (same box, rotated weights: M 2048 x N 12288 x K 5120
    // 118.1 -> 123.7 us, M 8192 x N 5120 x K 5120 184.5 -> 192.0): the pieces of the whole round's CUs all finish
    // together and write their partials in one burst, where 512 quarter tiles run two per CU
    if (s < 2 || (s == 2 && *full > 0)) return 1;
    // after whole rounds, pieces shorter than 32 stages tie or lose (same box: M 4096 x N 9472 x K 6144, 80 x 3 of 16
    // stages, 222.4 us against 215.8; M 1536 x N 14336 x K 6144 135.8 against 134.7); the MLP down projection's 64 x 4
    // of 34 stages wins (313.8 -> 299.4 us)
    if (*full > 0 && nk / s < 32) return 1;
    // where the quarter tiles run one per CU with 4 stages (4 rem <= CUs) they take ~0.42 of a whole tile's time
    // (~nk + 8 stages); a piece takes nk / s stages plus ~8 stages of fixed cost.  Same box: M 1000 x N 3000 x
    // K 4112 (48 x 2) 24.7 us as quarter tiles against 31.9 split; M 4096 x N 17152 x K 6144 (48 x 3 after whole
    // rounds) 353.1 against 359.4; M 300 x N 1000 x K 17408 (8 x 8) 76.8 against 44.9
    if (4 * *rem <= cus && 100 * (nk / s + 8) >= 42 * (nk + 8)) return 1;
    *bytes = (long)SPLIT_HEAD_INTS * 4 + (long)*rem * s * SPLIT_SLOT_INTS * 4;
    return s;
}

// K split of the 64 x 64 mid tiles (33..256 rows, with a workspace).  Against more than 12288 weight rows a workgroup
// is bound by its own stage loop rather than by HBM (at M = 64, K = 5120 the time grows ~20 us + bytes / 8.8 TB/s with
// N), so two K pieces per tile halve each workgroup's loop where both pieces of every tile fit at two workgroups per CU
// (64 KB of LDS each).  Same box, rotated weights, bf16 with bias, unsplit -> split: M 64 x N 16384 34.0 -> 25.2 us, M
// 64 x N 12800 33.6 -> 23.8, M 48 x N 13312 30.8 -> 22.8, M 64 x N 13312 x K 17408 93.1 -> 59.8, M 64 x N 17408 (272
// tiles) 35.1 -> 32.1, M 40 x N 17408 x K 17408 85.4 -> 76.0; three pieces tie with two at 272 tiles and lose up to 17%
// below, four to eight lose more; more tiles than that lose (M 64 x N 24576 36.4 -> 41.0, M 128 x N 17408 42.3 ->
// 45.1), and 3 K stages (three workgroups per CU) run the unsplit tiles 40% slower and the split ones no faster.
// More tiles than CUs: 2 (tiles - CUs) of them split unevenly (gemm_kernel's KSPLIT mapping), so that the first round
// of two workgroups per CU holds both halves of the others and a long first piece of these, and their short pieces
// run on the slots the halves free; that takes the split up to 5/4 tiles per CU.  Same box, equal halves -> uneven:
// M 64 x N 17408 x K 5120 (272 tiles) 32.6 -> 29.8 us, M 33 x N 17408 28.9 -> 26.7, M 40 x N 17408 x K 17408
// 75.5 -> 72.8; unsplit -> uneven: M 64 x N 20480 (320 tiles) 35.5 -> 32.1; past 5/4 it loses (M 48 x N 22528, 352
// tiles, 33.5 -> 34.0; M 64 x N 24576 37.1 -> 37.9).
#ifndef W8_MID_SPLIT
#define W8_MID_SPLIT -1                                  // -1: mid_split_plan's choice; 0 or 1: none; s >= 2: s pieces
#endif
#ifndef W8_MID_UNEVEN
#define W8_MID_UNEVEN 1                                  // 0: equal halves only, up to 17/16 tiles per CU
#endif
// At most 12288 weight rows (where, without a workspace, the streaming passes or the 64 x 128 tiles run): as many
// pieces per tile as fill two workgroups per CU once, min(2 CUs / tiles, stages / 16, 8), where N > 4096 or K has at
// least 64 stages.  Same box, rotated weights, bf16 with bias, without -> with the split: M 64 x N 12288 x K 5120
// 33.7 -> 24.7 us, M 33 x N 12288 27.3 -> 21.4, M 64 x N 10240 32.5 -> 23.7, M 64 x N 8192 18.3 -> 15.6, M 40 x
// N 6144 14.7 -> 13.7, M 64 x N 5120 x K 5120 17.2 -> 14.4, M 64 x N 5120 x K 17408 37.8 -> 31.0, M 48 x N 6144 x
// K 17408 34.0 -> 31.8, M 64 x N 1024 x K 17408 26.0 -> 20.1, M 64 x N 6144 x K 4096 14.8 -> 11.9; at 65..128 rows,
// where the streaming passes read the weights twice, M 128 x N 5120 x K 17408 74.9 -> 37.2, M 96 64.5 -> 34.1,
// M 128 x N 8192 x K 5120 35.4 -> 21.4, M 128 x N 6144 34.8 -> 20.6, M 100 x N 5120 x K 5120 31.2 -> 18.8.  At
// N <= 4096 with fewer stages the streaming passes stay faster (M 64 x N 4096 x K 5120 12.0 against 13.5, N 2048
// 11.3 against 12.9, M 48 x N 3072 10.7 against 12.7); M 128 x N 12288 (384 tiles) gets one piece and keeps the
// 64 x 128 tiles (26.8 us either way).
// 129..256 rows against at most 8192 weight rows (the 64 x 128 tiles' range above 128 rows) split the same way where
// K has at least 64 stages: M 192 x N 5120 x K 17408 65.3 -> 46.5 us, M 160 60.4 -> 44.5, M 256 x N 4096 x K 17408
// 63.8 -> 45.3; with 40 stages they lose (M 256 x N 5120 x K 5120 24.2 against 25.7, M 160 x N 6144 23.5 against
// 24.4), and two uneven pieces past one tile per CU tie or lose here (M 256 x N 5120 x K 17408 64.9 / 64.5, M 128 x
// N 10240 x K 5120 26.7 / 27.5).
static bool mid64_path(int M, int N, int K) {
    const int nk = (K + 127) / 128;
    if (M <= 32) return false;
    if (M <= MID_GEMM_MAX_M) return N > 4096 || nk >= 64;
    return M <= 2 * MID_GEMM_MAX_M && N <= 8192 && nk >= 64;
}
static int mid_split_plan(int M, int N, int K, int cus, long* bytes, int* uneven = nullptr) {
    *bytes = 0;
    if (uneven) *uneven = 0;
    if (!mid64_path(M, N, K)) return 1;
    const int tiles = ((M + 63) / 64) * ((N + 63) / 64), nk = (K + 127) / 128;
    int s = W8_MID_SPLIT;
    if (s < 0 && N <= MID_GEMM_WIDE_N) s = min(min(2 * cus / tiles, nk / 16), SPLIT_MAX);
    // wider: two pieces where they fit two workgroups per CU in about one round (64 KB of LDS each) and stay >= 16
    // stages
    if (s < 0) s = (W8_MID_UNEVEN ? 4 * tiles <= 5 * cus : 16 * tiles <= 17 * cus) && nk >= 32 ? 2 : 1;
    // at most 4096 slots of 16 KB, so that any plan fits the allocation-free entry's scratch (64 MiB of slots)
    s = min(min(s, nk), 4096 / tiles);
    if (s < 2 || tiles > SPLIT_HEAD_INTS) return 1;
    if (uneven && W8_MID_UNEVEN && s == 2 && tiles > cus) *uneven = min(2 * (tiles - cus), tiles);
    *bytes = (long)SPLIT_HEAD_INTS * 4 + (long)tiles * s * 64 * 64 * 4;
    return s;
}

template <typename T, int EPI>
static void launch_gemm(const Args& p, int policy = W8_GEMM_POLICY) {
    if (policy == 1 && p.ws) {                           // the K splits, when the caller gave a workspace
        long mbytes;
        int uneven;
        const int ms = mid_split_plan(p.M, p.N, p.K, cu_count(), &mbytes, &uneven);
        if (ms >= 2 && mbytes <= p.ws_bytes) {
            const int tiles = ((p.M + 63) / 64) * ((p.N + 63) / 64);
            launch_gemm_cfg<T, EPI, Mid64Cfg, true>(p, uneven, tiles * ms, ms);
            return;
        }
        int full, rem;
        long bytes;
        const int s = split_plan(p.M, p.N, p.K, cu_count(), &full, &rem, &bytes);
        if (s >= 2 && bytes <= p.ws_bytes) {
            // whole rounds before the last as their own launch; the last whole round and the pieces as one, so that
            // the pieces start on each CU as its whole tile ends
            const int cus = cu_count(), lead = full > cus ? full - cus : 0;
            if (lead > 0) launch_gemm_pp<T, EPI>(p, 0, lead);
            launch_gemm_pp_split<T, EPI>(p, lead, full - lead, rem, s);
            return;
        }
    }
    if (policy == 1 && mid_stream(p.M, p.N)) {
        launch_stream_rows<T, EPI>(p);
        return;
    }
    const int tiles = ((p.M + SUPER - 1) / SUPER) * ((p.N + SUPER - 1) / SUPER);
    if (policy == 1 && (p.M <= MID_GEMM_MAX_M || (p.M <= 2 * MID_GEMM_MAX_M && p.N <= 8192))) {
        if (p.N <= MID_GEMM_WIDE_N) {
            constexpr int SUBM = GemmCfg<MidCfg::WM, MidCfg::WN, MidCfg::FM, MidCfg::FN, MidCfg::KB, MidCfg::NS>::SUB;
            launch_gemm_cfg<T, EPI, MidCfg>(p, 0, tiles * SUBM);
        } else {
            constexpr int SUB6 =
                GemmCfg<Mid64Cfg::WM, Mid64Cfg::WN, Mid64Cfg::FM, Mid64Cfg::FN, Mid64Cfg::KB, Mid64Cfg::NS>::SUB;
            launch_gemm_cfg<T, EPI, Mid64Cfg>(p, 0, tiles * SUB6);
        }
        return;
    }
    constexpr int SUB =
        GemmCfg<SmallCfg::WM, SmallCfg::WN, SmallCfg::FM, SmallCfg::FN, SmallCfg::KB, SmallCfg::NS>::SUB;
    if (policy == 2) {
        launch_gemm_cfg<T, EPI, SmallCfg>(p, 0, tiles * SUB);
        return;
    }
    const int cus = cu_count();
    const int full = tiles / cus * cus, rem = tiles - full;
    const bool longk = tiles >= LONG_ROUNDS * cus;
    const bool pp = policy == 3 || (W8_GEMM_PP && policy != 0);
    if (policy == 0 || policy == 3 || rem == 0 || rem > cus / W8_SMALL_REM_DIV) {
        if (pp) launch_gemm_pp<T, EPI>(p, 0, tiles);
        else if (longk) launch_gemm_cfg<T, EPI, LongCfg>(p, 0, tiles);
        else launch_gemm_cfg<T, EPI, MainCfg>(p, 0, tiles);
        return;
    }
    if (full > 0 && pp) launch_gemm_pp<T, EPI>(p, 0, full);
    else if (full > 0 && longk) launch_gemm_cfg<T, EPI, LongCfg>(p, 0, full);
    else if (full > 0) launch_gemm_cfg<T, EPI, MainCfg>(p, 0, full);
    // the remainder as quarter tiles: with 4 K stages where they fit in one round at one workgroup per CU, else with 2
    // (two workgroups per CU)
    if (rem * SUB <= cus) launch_gemm_cfg<T, EPI, SmallDeepCfg>(p, full, rem * SUB);
    else launch_gemm_cfg<T, EPI, SmallCfg>(p, full, rem * SUB);
}

template <int EPI>
static void dispatch_dtype_stream(const Args& p, int dtype) {
    if (dtype == DT_F16) launch_stream<f16, EPI>(p);
    else launch_stream<bf16, EPI>(p);
}
template <int EPI>
static void dispatch_dtype_gemm(const Args& p, int dtype) {
    if (dtype == DT_F16) launch_gemm<f16, EPI>(p);
    else launch_gemm<bf16, EPI>(p);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static int check_common(const void* a, const void* w, int M, int N, int K, int dtype) {
    if (M < 1 || N < 1 || K < 16 || (K & 15) != 0 || K >= 131072) return -1;
    if ((long)M * K >= (1L << 31) || (long)N * K >= (1L << 31)) return -1;    // 32-bit buffer offsets
    if (dtype != DT_F16 && dtype != DT_BF16) return -1;
    if (!aligned16(a) || !aligned16(w)) return -1;
    return 0;
}

}  // namespace w8

using namespace w8;

// The small-M paths.  Same arguments as csrc/w8a8_gemv.cu:347 / :330: a [M, K] int8, w [N, K] int8, sa float32
// [M] (sa_rows = 1) or [1], sw float32 [N] (sw_rows = 1) or [1], bias [N] of the output type or null, out [M, N];
// dtype 0 = fp16, 1 = bf16.  Returns -1 on bad arguments, else the HIP error code of the launch (0 = success).
extern "C" int w8a8_gemv(const void* a, const void* w, const void* sa, const void* sw, const void* bias, void* out,
                         int M, int N, int K, int sa_rows, int sw_rows, int dtype, void* stream) {
    if (M > 16 || check_common(a, w, M, N, K, dtype) != 0) return -1;
    const Args p{(const int8_t*)a, (const int8_t*)w, (const float*)sa, (const float*)sw, (const uint16_t*)bias, out,
                 M, N, K, sa_rows, sw_rows, (hipStream_t)stream};
    dispatch_dtype_stream<EPI_SMALL>(p, dtype);
    return (int)hipGetLastError();
}

extern "C" int w8a8_mma(const void* a, const void* w, const void* sa, const void* sw, const void* bias, void* out,
                        int M, int N, int K, int sa_rows, int sw_rows, int dtype, void* stream) {
    if (M > 32 || check_common(a, w, M, N, K, dtype) != 0) return -1;
    const Args p{(const int8_t*)a, (const int8_t*)w, (const float*)sa, (const float*)sw, (const uint16_t*)bias, out,
                 M, N, K, sa_rows, sw_rows, (hipStream_t)stream};
    dispatch_dtype_stream<EPI_SMALL>(p, dtype);
    return (int)hipGetLastError();
}

// w8a8_gemv from 16-bit activations: x [M, K] fp16 / bf16 (dtype, also the output type; row stride ldx elements) is
// quantized per token (per_token_quant's arithmetic) and multiplied with the small-M epilogue; the int8 rows and
// their scales are also written to xq [M, K] and xs [M].  At one row within the VALU GEMV's K limit (x 16-byte
// aligned, ldx % 8 == 0) each workgroup quantizes the row itself, otherwise per_token_quant runs first.
// No counterpart in the reference (whose quantization is fused into the producer by inductor, quantfuse.py:1-10).
extern "C" int w8a8_gemv_quant(const void* x, long ldx, void* xq, void* xs, const void* w, const void* sw,
                               const void* bias, void* out, int M, int N, int K, int sw_rows, int dtype,
                               void* stream) {
    if (M > 16 || !x || !xq || !xs || ldx < K || check_common(xq, w, M, N, K, dtype) != 0) return -1;
    Args p{(const int8_t*)xq, (const int8_t*)w, (const float*)xs, (const float*)sw, (const uint16_t*)bias, out, M, N,
           K, 1, sw_rows, (hipStream_t)stream};
    // one row only: at two rows the 4-wavefront grid the shared quantization needs loses to the 1-wavefront grid of
    // the plain GEMV by more than the separate quantization costs (K = 6144, N = 5120: 12.0 against 9.6 us; at one row
    // 9.3 against 9.2 us, at N = 16384 16.0 against 16.4 us)
    if (M == 1 && dot4_ok(p) && (uintptr_t)x % 16 == 0 && ldx % 8 == 0) {
        p.x = static_cast<const uint16_t*>(x);
        p.ldx = ldx;
        p.xq = static_cast<int8_t*>(xq);
        p.xs = static_cast<float*>(xs);
        if (dtype == DT_F16) launch_dot4<f16, EPI_SMALL, true>(p);
        else launch_dot4<bf16, EPI_SMALL, true>(p);
        return (int)hipGetLastError();
    }
    const int rc = per_token_quant(x, xq, xs, M, K, ldx, dtype, stream);
    if (rc != 0) return rc;
    dispatch_dtype_stream<EPI_SMALL>(p, dtype);
    return (int)hipGetLastError();
}

// The decode MLP's gate_up GEMV with SiLU * up in its epilogue: w [2I, K] (gate rows, then up rows), h [M, I] =
// silu(g) * u as silu_mul_quant forms it before quantizing (g, u rounded as w8a8_gemv writes them), so that
// per_token_quant(h) equals silu_mul_quant(w8a8_gemv output) bit for bit.  Taken where the VALU GEMV takes M and K
// (M <= 5; K <= 17408 at one row, 8192 at two or three, 5120 at four or five): 1 = cannot implement otherwise.
// No counterpart in the reference (whose MLP runs the GEMV and silu_quant.cu:71 as two launches).
extern "C" int w8a8_gemv_silu(const void* a, const void* w, const void* sa, const void* sw, const void* bias, void* h,
                              int M, int I, int K, int sa_rows, int sw_rows, int dtype, void* stream) {
    if (I < 1 || M > 16 || check_common(a, w, M, 2 * I, K, dtype) != 0 || !h) return -1;
    const Args p{(const int8_t*)a, (const int8_t*)w, (const float*)sa, (const float*)sw, (const uint16_t*)bias, h, M,
                 I, K, sa_rows, sw_rows, (hipStream_t)stream};
    if (!dot4_ok(p)) return 1;
    if (dtype == DT_F16) launch_dot4_silu<f16>(p);
    else launch_dot4_silu<bf16>(p);
    return (int)hipGetLastError();
}

// The prefill path: csrc/w8a8_big.cu:66 arguments (per-row sa [M], per-column sw [N], no bias).  Return codes as
// there: 0 ok, 1 cannot implement (shape / alignment), 3 launch failed.
extern "C" int w8a8_big(const void* A, const void* W, const void* sa, const void* sw, void* out, int M, int N, int K,
                        int dtype, void* stream) {
    if (check_common(A, W, M, N, K, dtype) != 0 || (N & 15) != 0) return 1;
    const Args p{(const int8_t*)A, (const int8_t*)W, (const float*)sa, (const float*)sw, nullptr, out, M, N, K, 1, 1,
                 (hipStream_t)stream};
    dispatch_dtype_gemm<EPI_LARGE>(p, dtype);
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

// Every shape the reference hands to vLLM's cutlass_scaled_mm fallback (vllm_turing/w8a8.py:117): any M, optional
// bias, per-row or per-tensor scales, with that op's large-M epilogue (csrc/w8a8_big.cu:26-35; with a bias
// fma(sa, RN32(acc * sw), b)).  M <= 32 runs the streaming kernel, larger M the prefill kernel.
// Returns -1 on bad arguments, else the HIP error code of the launch.
extern "C" int w8a8_scaled_mm(const void* a, const void* w, const void* sa, const void* sw, const void* bias,
                              void* out, int M, int N, int K, int sa_rows, int sw_rows, int dtype, void* stream) {
    if (check_common(a, w, M, N, K, dtype) != 0) return -1;
    const Args p{(const int8_t*)a, (const int8_t*)w, (const float*)sa, (const float*)sw, (const uint16_t*)bias, out,
                 M, N, K, sa_rows, sw_rows, (hipStream_t)stream};
    if (M <= 32) {
        if (bias) dispatch_dtype_stream<EPI_LARGE_BIAS>(p, dtype);
        else dispatch_dtype_stream<EPI_LARGE>(p, dtype);
    } else {
        if (bias) dispatch_dtype_gemm<EPI_LARGE_BIAS>(p, dtype);
        else dispatch_dtype_gemm<EPI_LARGE>(p, dtype);
    }
    return (int)hipGetLastError();
}

// Workspace bytes w8a8_scaled_mm_ws takes for M x N x K on the current device (0: that shape does not split); -1 on
// bad sizes.
extern "C" long w8a8_scaled_mm_ws_size(int M, int N, int K) {
    if (M < 1 || N < 1 || K < 16) return -1;
    int full, rem;
    long bytes, mbytes;
    split_plan(M, N, K, cu_count(), &full, &rem, &bytes);
    mid_split_plan(M, N, K, cu_count(), &mbytes);
    return max(bytes, mbytes);
}

// w8a8_scaled_mm with a workspace (16-byte aligned, ws_bytes >= w8a8_scaled_mm_ws_size(M, N, K); its first 4 KB zero
// before the first call, and every call leaves them zero) for the prefill GEMM's K splits (split_plan for a last
// partial round of super tiles, mid_split_plan for the 64 x 64 tiles of 33..64 rows); dtype 2
// writes the raw int32 accumulators to out [M, N] instead (sa, sw, bias unused).  Calls that share a workspace must
// not overlap.  Returns -1 on bad arguments (a workspace too small included), else the HIP error of the launches.
extern "C" int w8a8_scaled_mm_ws(const void* a, const void* w, const void* sa, const void* sw, const void* bias,
                                 void* out, int M, int N, int K, int sa_rows, int sw_rows, int dtype, void* workspace,
                                 long ws_bytes, void* stream) {
    const bool raw = dtype == 2;
    if (check_common(a, w, M, N, K, raw ? DT_F16 : dtype) != 0) return -1;
    const long need = w8a8_scaled_mm_ws_size(M, N, K);
    if (need > 0 && (!workspace || ws_bytes < need || ((uintptr_t)workspace & 15) != 0)) return -1;
    Args p{(const int8_t*)a, (const int8_t*)w, (const float*)sa, (const float*)sw, (const uint16_t*)bias, out, M, N,
           K, sa_rows, sw_rows, (hipStream_t)stream};
    p.ws = static_cast<int*>(workspace);
    p.ws_bytes = ws_bytes;
    if (raw) {
        launch_gemm<f16, EPI_I32>(p);
    } else if (M <= 32) {
        if (bias) dispatch_dtype_stream<EPI_LARGE_BIAS>(p, dtype);
        else dispatch_dtype_stream<EPI_LARGE>(p, dtype);
    } else {
        if (bias) dispatch_dtype_gemm<EPI_LARGE_BIAS>(p, dtype);
        else dispatch_dtype_gemm<EPI_LARGE>(p, dtype);
    }
    return (int)hipGetLastError();
}

// ---- w8a8_scaled_mm_noalloc: w8a8_scaled_mm_ws with the library's own scratch in place of the workspace ------------
// For callers that cannot allocate (HIP graph capture, serving loops that forbid allocation).  The scratch is a
// file-scope device array: 4 KB of tile counters and 256 accumulator slots of 256 KB (64 MiB + 4 KiB), enough for the
// K split of any shape on a GPU of up to 256 CUs (a larger need is rejected).  Each GPU the library runs on holds its
// own copy until the process ends; every call on a GPU shares it, so calls that overlap on one GPU (other streams,
// other threads) race.  In host code `scratch` only names the host-side stand-in of the array: its device address
// comes from hipGetSymbolAddress, once per device, and is what the kernels get.
constexpr long NOALLOC_SLOTS = 256;
constexpr long NOALLOC_SCRATCH_INTS = SPLIT_HEAD_INTS + NOALLOC_SLOTS * SPLIT_SLOT_INTS;
static __device__ __align__(256) int scratch[NOALLOC_SCRATCH_INTS];

__global__ void __launch_bounds__(256) clear_ints_kernel(int* __restrict__ p, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

// The device address of this device's scratch (null on failure).  The first call on a device also clears the tile
// counters with a kernel on `st` (the loader's zero fill of the array is not relied on); a call under stream capture
// records that clear in the graph (harmless: the counters are zero whenever no call runs) and leaves the eager clear
// to the next call outside capture.
static int* scratch_setup(hipStream_t st) {
    constexpr int MAX_DEV = 64;
    static std::atomic<int*> addr[MAX_DEV];
    static std::atomic<bool> cleared[MAX_DEV];
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return nullptr;
    int* p = addr[dev].load(std::memory_order_acquire);
    if (!p) {
        void* q = nullptr;
        if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || !q) return nullptr;
        p = static_cast<int*>(q);
        addr[dev].store(p, std::memory_order_release);
    }
    if (!cleared[dev].load(std::memory_order_acquire)) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        const bool capturing = hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone;
        clear_ints_kernel<<<1, 256, 0, st>>>(p, SPLIT_HEAD_INTS);
        if (hipGetLastError() != hipSuccess) return nullptr;
        if (!capturing) cleared[dev].store(true, std::memory_order_release);
    }
    return p;
}

// w8a8_scaled_mm_ws's arguments without the workspace.  Returns -1 on bad arguments, -2 when the shape's K split
// would need more than the scratch holds, -3 when the scratch's address cannot be had, else the HIP error of the
// launches.  Allocates nothing.
extern "C" int w8a8_scaled_mm_noalloc(const void* a, const void* w, const void* sa, const void* sw, const void* bias,
                                      void* out, int M, int N, int K, int sa_rows, int sw_rows, int dtype,
                                      void* stream) {
    if (check_common(a, w, M, N, K, dtype == 2 ? DT_F16 : dtype) != 0) return -1;
    const long need = w8a8_scaled_mm_ws_size(M, N, K);
    if (need < 0) return -1;
    if (need > NOALLOC_SCRATCH_INTS * 4) return -2;
    int* ws = nullptr;
    if (need > 0 && !(ws = scratch_setup((hipStream_t)stream))) return -3;
    return w8a8_scaled_mm_ws(a, w, sa, sw, bias, out, M, N, K, sa_rows, sw_rows, dtype, ws,
                             ws ? NOALLOC_SCRATCH_INTS * 4 : 0, stream);
}

// Test export: the raw int32 accumulators acc [M, N] of one kernel's main loop (kernel 0 = the MFMA streaming kernel,
// M <= 64; kernel 1 = the prefill kernel as dispatched; kernel 2 = the VALU dot4 kernel, M = 1 and K <= 17408,
// M = 2, 3 and K <= 8192, M = 4, 5 and K <= 5120; kernel 3 = the prefill kernel's quarter-tile configuration alone;
// kernel 4 = its full-tile configuration alone).  Returns -1 on bad arguments, else the launch error.
extern "C" int w8a8_i32(const void* a, const void* w, void* acc, int M, int N, int K, int kernel, void* stream) {
    if (check_common(a, w, M, N, K, DT_F16) != 0 || kernel < 0 || kernel > 5) return -1;
    const Args p{(const int8_t*)a, (const int8_t*)w, nullptr, nullptr, nullptr, acc, M, N, K, 0, 0,
                 (hipStream_t)stream};
    if (kernel == 0) {
        if (M > 64) return -1;
        if (M <= 16) launch_stream_lds<f16, 1, EPI_I32>(p);
        else if (M <= 32) launch_stream_lds<f16, 2, EPI_I32>(p);
        else launch_stream_lds<f16, 4, EPI_I32>(p);
    } else if (kernel == 1) {
        launch_gemm<f16, EPI_I32>(p);
    } else if (kernel == 3) {
        launch_gemm<f16, EPI_I32>(p, 2);
    } else if (kernel == 4) {
        launch_gemm<f16, EPI_I32>(p, 0);
    } else if (kernel == 5) {
        launch_gemm<f16, EPI_I32>(p, 3);
    } else {
        if (!dot4_ok(p)) return -1;
        launch_dot4<f16, EPI_I32>(p);
    }
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------------
// hbm_read: the M = 1 GEMV's weight stream without its math (the ceiling the GEMV is measured against)
// ---------------------------------------------------------------------------------------------------------------------
// Rows of K bytes exactly as gemv_dot4_kernel reads them at one activation row: one-wavefront workgroups, rows
// grid-strided over ceil(rows / 3) wavefronts, each wavefront instruction 1 KB of one row (lane l: 16-byte chunks l,
// l + 64, ...), non-temporal, the next row's loads issued before the current row is consumed.  The words are XORed
// and the result stored only if it equals a value no real input produces in practice, so nothing is written while
// the loads cannot be removed.
template <int CH>
__global__ void __launch_bounds__(64) hbm_read_kernel(const int8_t* __restrict__ src, int rows, int K,
                                                      int* __restrict__ sink) {
    const int lane = threadIdx.x & 63, nw = gridDim.x, wid = blockIdx.x, K16 = K >> 4;
    if (wid >= rows) return;
    v4i buf[2][CH];
    auto load = [&](int b, int r) {
        const int8_t* row = src + (long)min(r, rows - 1) * K;
#pragma unroll
        for (int j = 0; j < CH; ++j) buf[b][j] = wload<true>(row + min(lane + 64 * j, K16 - 1) * 16);
    };
    int x = 0;
    auto use = [&](int b) {
#pragma unroll
        for (int j = 0; j < CH; ++j) x ^= buf[b][j].x ^ buf[b][j].y ^ buf[b][j].z ^ buf[b][j].w;
    };
    const int cnt = (rows - 1 - wid) / nw + 1;
    load(0, wid);
    int k = 0;
    for (; k + 2 < cnt; k += 2) {                        // peeled and fenced as gemv_dot4_kernel
        load(1, wid + (k + 1) * nw);
        __builtin_amdgcn_sched_barrier(0);               // the loads stay ahead of the use
        use(0);
        load(0, wid + (k + 2) * nw);
        __builtin_amdgcn_sched_barrier(0);               // the loads stay ahead of the use
        use(1);
    }
    if (k + 1 < cnt) {
        load(1, wid + (k + 1) * nw);
        __builtin_amdgcn_sched_barrier(0);               // the loads stay ahead of the use
        use(0);
        use(1);
    } else {
        use(0);
    }
    if (x == 0x5a3c96e1) sink[0] = x;
}

// ---------------------------------------------------------------------------------------------------------------------
// W8A16 (int8 LM head)
// ---------------------------------------------------------------------------------------------------------------------
// M = 1 up to K = 8192 and M = 2 up to K = 5120 (the activations' registers) take the VALU kernel.  Three rows take
// fewer wavefronts per SIMD and tie with the MFMA kernel in bf16 (N = 248320, K = 5120: 219.5 against 218.3 us) and
// lose in fp16 (227.8 against 216.4 us); four rows take 256 registers, one wavefront per SIMD, and lose by more.
constexpr int W8A16_DOT_MAX_CH_M1 = 8, W8A16_DOT_MAX_CH_M2 = 5;

template <typename T, int M, int CH, bool GATHER>
static void launch_w8a16_dot_t(const void* x, const void* w, const void* s, const void* bias, void* out, int N, int K,
                               int w_rows, const int* rows, hipStream_t st) {
    static const int per_cu = row_stream_per_cu(reinterpret_cast<const void*>(&w8a16_dot_kernel<T, M, CH, GATHER>));
    const int need = (N + 3) / 4, grid = cu_count() * per_cu;
    w8a16_dot_kernel<T, M, CH, GATHER><<<need < grid ? need : grid, 256, 0, st>>>(
        static_cast<const uint16_t*>(x), static_cast<const int8_t*>(w), static_cast<const float*>(s),
        static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), N, K, w_rows, rows);
}
template <typename T, int M, bool GATHER>
static bool launch_w8a16_dot_m(const void* x, const void* w, const void* s, const void* bias, void* out, int N, int K,
                               int w_rows, const int* rows, hipStream_t st) {
    const int ch = (K / 16 + 63) / 64;
    if (ch > (M == 1 ? W8A16_DOT_MAX_CH_M1 : W8A16_DOT_MAX_CH_M2)) return false;
    switch (ch) {
#define W8_CASE(C) case C: if constexpr (M == 1 || C <= W8A16_DOT_MAX_CH_M2) \
            launch_w8a16_dot_t<T, M, C, GATHER>(x, w, s, bias, out, N, K, w_rows, rows, st); break;
        W8_CASE(1) W8_CASE(2) W8_CASE(3) W8_CASE(4) W8_CASE(5) W8_CASE(6) W8_CASE(7) W8_CASE(8)
#undef W8_CASE
        default: return false;
    }
    return true;
}
template <typename T>
static bool launch_w8a16_dot(const void* x, const void* w, const void* s, const void* bias, void* out, int M, int N,
                             int K, int w_rows, const int* rows, hipStream_t st) {
    if (M == 1) return rows ? launch_w8a16_dot_m<T, 1, true>(x, w, s, bias, out, N, K, w_rows, rows, st)
                            : launch_w8a16_dot_m<T, 1, false>(x, w, s, bias, out, N, K, w_rows, rows, st);
    if (M == 2) return rows ? launch_w8a16_dot_m<T, 2, true>(x, w, s, bias, out, N, K, w_rows, rows, st)
                            : launch_w8a16_dot_m<T, 2, false>(x, w, s, bias, out, N, K, w_rows, rows, st);
    return false;
}

// Several 16-row weight tiles per workgroup share each activation fragment (the activations are re-read from L2 by
// every workgroup: at M = 16, 4 KB per 128-byte K step against 2 KB of weights), all weight loads non-temporal.
// N = 248320, K = 5120, bf16, against one tile: two tiles M=4 251 -> 226 us, M=8 288 -> 240, M=16 378 -> 290, M=32
// 730 -> 445; three tiles (72 KB rings, two workgroups per CU) M=4 248, M=8 262, M=16 291, M=32 379 us; four tiles
// (one workgroup per CU) lose at M <= 16.  So two tiles up to M = 16 and three above.
template <typename T, int MT, bool GATHER>
static void launch_w8a16_t(const void* x, const void* w, const void* s, const void* bias, void* out, int M, int N,
                           int K, int w_rows, const int* rows, hipStream_t st) {
    constexpr int NS = 3, RT = MT == 1 ? 2 : 3, LDS = 4 * NS * RT * 16 * 128;
    static_assert(LDS >= 3 * RT * MT * 4 * 64 * 4, "the K-slice reduction fits in the rings");
    const void* kern = reinterpret_cast<const void*>(&w8a16_kernel<T, MT, NS, GATHER, RT>);
    static const hipError_t attr = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, LDS);
    (void)attr;
    w8a16_kernel<T, MT, NS, GATHER, RT><<<(N + 16 * RT - 1) / (16 * RT), 256, LDS, st>>>(
        static_cast<const uint16_t*>(x), static_cast<const int8_t*>(w), static_cast<const float*>(s),
        static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), M, N, K, w_rows, rows);
}
template <typename T>
static void launch_w8a16(const void* x, const void* w, const void* s, const void* bias, void* out, int M, int N, int K,
                         int w_rows, const int* rows, hipStream_t st) {
    if (launch_w8a16_dot<T>(x, w, s, bias, out, M, N, K, w_rows, rows, st)) return;
    if (M <= 16) {
        if (rows) launch_w8a16_t<T, 1, true>(x, w, s, bias, out, M, N, K, w_rows, rows, st);
        else launch_w8a16_t<T, 1, false>(x, w, s, bias, out, M, N, K, w_rows, rows, st);
    } else {
        if (rows) launch_w8a16_t<T, 2, true>(x, w, s, bias, out, M, N, K, w_rows, rows, st);
        else launch_w8a16_t<T, 2, false>(x, w, s, bias, out, M, N, K, w_rows, rows, st);
    }
}

static int w8a16_entry(const void* x, const void* w, const void* s, const void* bias, void* out, int M, int N, int K,
                       int dtype, int w_rows, const int* rows, void* stream) {
    if (M < 1 || M > 32 || N < 1 || K < 16 || (K & 15) != 0 || w_rows < 1 || (long)w_rows * K >= (1L << 31)) return -1;
    if (dtype != DT_F16 && dtype != DT_BF16) return -1;
    if (!x || !w || !s || !out || (uintptr_t)x % 16 != 0 || (uintptr_t)w % 16 != 0) return -1;
    hipStream_t st = (hipStream_t)stream;
    if (dtype == DT_F16) launch_w8a16<f16>(x, w, s, bias, out, M, N, K, w_rows, rows, st);
    else launch_w8a16<bf16>(x, w, s, bias, out, M, N, K, w_rows, rows, st);
    return (int)hipGetLastError();
}

// The int8 LM head (csrc/w8a16_gemv.cu:145-154, same arguments; M <= 32 here, against 16 there): out [M, N] of x [M, K]
// fp16 / bf16 (dtype 0 / 1) times the int8 rows w [N, K] with float32 per-row scales s [N] and an optional bias [N]
// of the activation type.  Returns -1 on bad arguments (M outside 1..32, K % 16, alignment), else the launch error.
extern "C" int w8a16_gemv(const void* x, const void* w, const void* s, const void* bias, void* out, int M, int N, int K,
                          int dtype, void* stream) {
    return w8a16_entry(x, w, s, bias, out, M, N, K, dtype, N, nullptr, stream);
}

// The same over a gathered subset of weight rows, with the reference's arguments (csrc/w8a16_gemv.cu:145-146,156-167):
// rows int32 [N] indexes rows of w and out [M, N] is compact over the subset; rows = null computes all N rows.  As
// there, every index must name a row of w (the caller's guarantee, e.g. a draft vocabulary built from the head): the
// library does not know w's row count, so indices are only clamped to the rows a 32-bit offset reaches
// (2^31 / K); w8a16_gemv_rows_bounded takes that count and clamps to it.
extern "C" int w8a16_gemv_rows(const void* x, const void* w, const void* s, const void* bias, void* out, int M, int N,
                               int K, int dtype, const void* rows, void* stream) {
    if (!rows) return w8a16_entry(x, w, s, bias, out, M, N, K, dtype, N, nullptr, stream);
    if (K < 16) return -1;
    const int reach = (int)(((1L << 31) - 1) / K);       // rows addressable by 32-bit buffer offsets
    return w8a16_entry(x, w, s, bias, out, M, N, K, dtype, reach, static_cast<const int*>(rows), stream);
}

// The gathered form with the row count of w: indices are clamped to [0, w_rows), so a bad index reads a row of w
// instead of memory past it.  No counterpart in the reference (whose rows are trusted).
extern "C" int w8a16_gemv_rows_bounded(const void* x, const void* w, const void* s, const void* bias, void* out, int M,
                                       int N, int K, int dtype, const void* rows, int w_rows, void* stream) {
    if (!rows) return -1;
    return w8a16_entry(x, w, s, bias, out, M, N, K, dtype, w_rows, static_cast<const int*>(rows), stream);
}

// The reference's tensor-core W8A16 entry (csrc/w8a16_mma.cu:176-191, same arguments and codes): x [M, K] fp16,
// w [N, K] int8, s [N] float32, bias [N] fp16 or null, out [M, N] fp16; 1 <= M <= 64 and N even, else -1; cfg 0 / 1 /
// other names the reference's k-tile of 128 / 256 / 512 bytes, and K must be a multiple of it (-1 otherwise); cfg
// with 512-byte k-tiles refuses M > 32 with -2 as the reference's shared-memory limit does.  Every cfg runs the same
// MFMA weight-streaming kernel here (in passes of at most 32 rows), so the outputs do not depend on cfg.  Also -1 on
// null or misaligned pointers (x and w 16-byte aligned).  Returns the launch error otherwise.
extern "C" int w8a16_mma(const void* x, const void* w, const void* s, const void* bias, void* out, int M, int N, int K,
                         int cfg, void* stream) {
    if (M < 1 || M > 64 || N % 2 != 0) return -1;
    const int kt = cfg == 0 ? 128 : cfg == 1 ? 256 : 512;
    if (K < kt || K % kt != 0) return -1;
    if (kt == 512 && M > 32) return -2;
    for (int r0 = 0; r0 < M; r0 += 32) {
        const int rows = M - r0 < 32 ? M - r0 : 32;
        const int rc = w8a16_entry(static_cast<const uint16_t*>(x) + (long)r0 * K, w, s, bias,
                                   static_cast<uint16_t*>(out) + (long)r0 * N, rows, N, K, DT_F16, N, nullptr, stream);
        if (rc != 0) return rc;
    }
    return 0;
}

// Test export: stream rows x K bytes of src (16-byte aligned, K % 16 == 0, K <= 17408) through the M = 1 GEMV's
// load path and discard them (sink: one int, written only in the improbable case described at hbm_read_kernel).  No
// counterpart in the reference.  Returns -1 on bad arguments, else the launch error.
extern "C" int hbm_read(const void* src, int rows, int K, void* sink, void* stream) {
    if (!src || !sink || rows < 1 || K < 16 || K % 16 != 0 || (uintptr_t)src % 16 != 0 || (long)rows * K >= (1L << 40))
        return -1;
    const int ch = dot4_chunks(K);
    const int waves = (rows + DOT4_ROWS_PER_WAVE - 1) / DOT4_ROWS_PER_WAVE;
    const int8_t* s8 = static_cast<const int8_t*>(src);
    int* sk = static_cast<int*>(sink);
    hipStream_t st = (hipStream_t)stream;
    switch (ch) {
#define W8_CASE(C) case C: hbm_read_kernel<C><<<waves, 64, 0, st>>>(s8, rows, K, sk); break;
        W8_CASE(1) W8_CASE(2) W8_CASE(3) W8_CASE(4) W8_CASE(5) W8_CASE(6) W8_CASE(7) W8_CASE(8) W8_CASE(10)
        W8_CASE(12) W8_CASE(14) W8_CASE(17)
#undef W8_CASE
        default: return -1;
    }
    return (int)hipGetLastError();
}
