/*
 * CPU oracle for the W8A8 SmoothQuant linear path.  TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C with IEEE single-precision arithmetic and no FMA contraction, the arithmetic of
 * cookjohn/vllm-turing's W8A8 path.  It is the checker the HIP kernels are compared against: only the tests, the
 * smoke check and the CPU-baseline leg of the benchmark load it.  The product library never links, loads or calls it.
 *
 * Every function cites the reference file:line it follows.  How each one is pinned (known answers, closed forms,
 * exhaustive tables, brute force) is stated beside it and exercised by tests/test_oracle_pins.py:
 *   o_quant_rows        pinned: closed form + invariants (|q|<=127, q=+-127 at the argmax, zero-row rule), and an
 *                       independent numpy restatement of quantfuse.py:18-24.
 *   o_gemm_i32          pinned: torch._int_mm (oneDNN) and a float64 matmul; brute force on tiny shapes.
 *   o_epilogue (small)  pinned: per-element restatement with numpy float32 + math.fma-free split, and the fp64
 *                       closed form of tests/test_w8a8_mma.py:43-51 within its tolerance.
 *   o_epilogue (large)  pinned: numpy float32 two-product chain; bias variant pinned only to tolerance (the
 *                       epilogue that defines it is vLLM's third-party cutlass_scaled_mm, absent here).
 *   o_silu_h            pinned: exhaustive 65,536-entry check against exp computed with Python's decimal module at
 *                       60 digits and correctly rounded to float32 (the reference's CUDA expf itself cannot be run or
 *                       reproduced; rare 1-ulp differences of CUDA's expf are the one unpinned residue).
 *   o_silu_mul_quant    pinned: composition of the above; the fp16 product is exact IEEE.
 *   o_w8a16             pinned: the float64 closed form (x . (w s)^T + bias) within one 16-bit rounding plus the float32
 *                       sum's error bound; gathered rows against the dense result; the sum order is the kernel's own
 *                       (float32 MFMA), so the GPU is compared to tolerance, as the reference's own head is.
 *   o_ar8_quant / o_ar8_dequant_sum
 *                       pinned: known groups (exact scales, ties to even, the -127 clamp, zero groups), invariants
 *                       (|q| <= 127, +-127 at each group's absmax, |x - q s| <= s / 2 in range), the dequantised sum
 *                       against exact rational arithmetic rounded once to fp16.
 *   o_rms_norm_quant    pinned: residual sum against numpy / torch IEEE conversion, the normalised row against the
 *                       float64 closed form within one 16-bit rounding, rms within 1.5 float32 ulps of the float64
 *                       value, known answers (constant rows -> +-127, zero row -> scale FLT_EPSILON and q = 0) and the
 *                       quant invariants.  Bit-level parity with vLLM's own op (third-party, absent; float32 block
 *                       sum and rsqrtf) is unpinned, see the function.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off -fno-fast-math; SSE2 float arithmetic on x86-64).
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

/* Contraction is disabled by the build (-ffp-contract=off); no fmaf appears except where the reference contracts. */

/* ------------------------------------------------------------------------------------------------------------------
 * fp16 / bf16 <-> fp32 conversions (IEEE round-to-nearest-even), written from the format definitions.
 * The reference converts with __half2float / __float2half_rn / __float2bfloat16_rn (csrc/w8a8_gemv.cu:12-17).
 * ------------------------------------------------------------------------------------------------------------------ */
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float o_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));          /* inf / nan */
    if (e == 0) {                                                         /* zero / subnormal: m * 2^-24, exact */
        float v = (float)m * u2f(0x33800000u);                            /* 2^-24 */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112) << 23) | (m << 13));
}

uint16_t o_f2h(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return sign | (a > 0x7f800000u ? 0x7e00 : 0x7c00);  /* nan / inf */
    if (a >= 0x477ff000u) return sign | 0x7c00;                  /* >= 65520 rounds to inf */
    if (a >= 0x38800000u) {                                      /* normal fp16 range: >= 2^-14 */
        uint32_t mant = a & 0x7fffff, exp = (a >> 23) - 112;
        uint32_t r = (exp << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fff;
        if (rem > 0x1000 || (rem == 0x1000 && (r & 1))) r++;     /* carry into the exponent is correct */
        return sign | (uint16_t)r;
    }
    /* subnormal fp16 (or zero): value / 2^-24 rounded to an integer, ties to even */
    float scaled = u2f(a) * 16777216.0f;                         /* exact: power-of-two scaling of a float */
    float fl = floorf(scaled);
    float rem = scaled - fl;                                     /* exact: scaled < 2^10 has >= 13 fraction bits */
    uint32_t r = (uint32_t)fl;
    if (rem > 0.5f || (rem == 0.5f && (r & 1))) r++;
    return sign | (uint16_t)r;                                   /* r == 1024 becomes the smallest normal: correct */
}

float o_bf2f(uint16_t b) { return u2f((uint32_t)b << 16); }

uint16_t o_f2bf(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);   /* quiet nan */
    uint32_t lsb = (u >> 16) & 1;
    u += 0x7fffu + lsb;                                          /* round to nearest even; overflow -> inf */
    return (uint16_t)(u >> 16);
}

static inline float to_f(uint16_t v, int dtype) { return dtype == 0 ? o_h2f(v) : o_bf2f(v); }
static inline uint16_t from_f(float v, int dtype) { return dtype == 0 ? o_f2h(v) : o_f2bf(v); }

/* ------------------------------------------------------------------------------------------------------------------
 * Round half to even of a float to an int8, saturating.
 * Follows csrc/silu_quant.cu:16-20 (rintf, fmaxf(-128), fminf(127)) and quantfuse.py:23 (torch.round half-even,
 * clamp(-128, 127)).  Inputs are finite in the path's contract (finite activations, see o_quant_rows).
 * ------------------------------------------------------------------------------------------------------------------ */
static inline int8_t q8(float v) {
    float r = rintf(v);                                          /* default rounding mode: nearest even */
    if (r < -128.0f) r = -128.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)r;
}

/* ------------------------------------------------------------------------------------------------------------------
 * Dynamic symmetric per-token int8 quantization of one row set.
 * Follows vllm_turing/quantfuse.py:18-24 (absmax in float32, scale = absmax / 127, q = round(x * (127 / absmax))
 * clamped) with the zero-row rule of csrc/silu_quant.cu:57-58 (absmax == 0 -> inverse 0, so q = 0 and scale = 0).
 * x: [M, K] fp16 (dtype 0) or bf16 (dtype 1) bit patterns with row stride ldx; q: [M, K] int8; s: [M] float32.
 * ------------------------------------------------------------------------------------------------------------------ */
void o_quant_rows(const uint16_t* x, int dtype, long M, long K, long ldx, int8_t* q, float* s) {
    for (long m = 0; m < M; ++m) {
        const uint16_t* xr = x + m * ldx;
        float amax = 0.0f;
        for (long k = 0; k < K; ++k) {
            float v = fabsf(to_f(xr[k], dtype));
            if (v > amax) amax = v;
        }
        const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        s[m] = amax / 127.0f;
        for (long k = 0; k < K; ++k) q[m * K + k] = q8(to_f(xr[k], dtype) * inv);
    }
}

/* ------------------------------------------------------------------------------------------------------------------
 * int8 x int8 -> int32 product acc[m, n] = sum_k a[m, k] * w[n, k].
 * Follows csrc/w8a8_gemv.cu:53-81 (dp4a sums over K, exact integer arithmetic) and csrc/w8a8_big.cu:36-43
 * (int32 accumulation; saturation can never trigger because |acc| <= 128*128*K < 2^31 for K < 131072).
 * a: [M, K] row-major; w: [N, K] row-major (the weight as stored; vLLM passes its [K, N] stride-(1, K) view).
 * Returns 0, or 1 if K is too large for the int32 bound above.
 * ------------------------------------------------------------------------------------------------------------------ */
int o_gemm_i32(const int8_t* a, const int8_t* w, int32_t* acc, long M, long N, long K) {
    if (K >= 131072) return 1;
    for (long m = 0; m < M; ++m) {
        const int8_t* ar = a + m * K;
        for (long n = 0; n < N; ++n) {
            const int8_t* wr = w + n * K;
            int32_t sum = 0;                                     /* exact: bound above */
            for (long k = 0; k < K; ++k) sum += (int32_t)ar[k] * (int32_t)wr[k];
            acc[m * N + n] = sum;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------------------------
 * Scale epilogue: int32 accumulators -> fp16 / bf16 output.
 * order 0, the small-M kernels (csrc/w8a8_gemv.cu:87-91 and :280-288):
 *     out = RN_T( fmaf( RN32(float(acc) * sa[m]), sw[n], b ) ),  b = float(bias[n]) or +0.0f
 *   The expression is `(float) acc * sa * sw + b`; nvcc's default --fmad=true contracts the last multiply-add.
 * order 1, the large-M kernel (csrc/w8a8_big.cu:26-35: ScaleB node first, then ScaleA, each rounded to float):
 *     out = RN_T( RN32( sa[m] * RN32(float(acc) * sw[n]) ) )
 *   and, with a bias (vLLM's c2x bias epilogue, third-party: multiply_add of ScaleA, the ScaleB product and Bias):
 *     out = RN_T( fmaf( sa[m], RN32(float(acc) * sw[n]), b ) )
 * sa has M entries when sa_rows else 1; sw has N entries when sw_rows else 1; bias may be NULL (same dtype as out).
 * ------------------------------------------------------------------------------------------------------------------ */
void o_epilogue(const int32_t* acc, const float* sa, const float* sw, const uint16_t* bias, uint16_t* out, long M,
                long N, int sa_rows, int sw_rows, int dtype, int order) {
    for (long m = 0; m < M; ++m) {
        const float sam = sa[sa_rows ? m : 0];
        for (long n = 0; n < N; ++n) {
            const float swn = sw[sw_rows ? n : 0];
            const float b = bias ? to_f(bias[n], dtype) : 0.0f;
            const float fa = (float)acc[m * N + n];
            float r;
            if (order == 0) {
                float t = fa * sam;
                r = fmaf(t, swn, b);
            } else {
                float t = fa * swn;
                r = bias ? fmaf(sam, t, b) : sam * t;
            }
            out[m * N + n] = from_f(r, dtype);
        }
    }
}

/* ------------------------------------------------------------------------------------------------------------------
 * SiLU of one fp16 (dtype 0) or bf16 (dtype 1) value, rounded back to that type.
 * Follows csrc/silu_quant.cu:11-14: f = float(x); RN_T( f / (1.0f + expf(-f)) ) with IEEE float division.  expf is
 * taken correctly rounded to float32: expl in x87 extended precision (64-bit significand), then rounded once to
 * float.  tests/test_oracle_pins.py checks every one of the 65,536 inputs of each type against a 60-digit decimal exp.
 * ------------------------------------------------------------------------------------------------------------------ */
static float expf_cr(float x) { return (float)expl((long double)x); }

uint16_t o_silu_h(uint16_t x, int dtype) {
    const float f = to_f(x, dtype);
    const float e = expf_cr(-f);
    const float d = 1.0f + e;
    return from_f(f / d, dtype);
}

/* The 65,536-entry silu table of one type (index = input bit pattern). */
void o_silu_table(int dtype, uint16_t* table) {
    for (uint32_t i = 0; i < 65536u; ++i) table[i] = o_silu_h((uint16_t)i, dtype);
}

/* ------------------------------------------------------------------------------------------------------------------
 * SiLU(gate) * up followed by per-row dynamic int8 quantization.
 * Follows csrc/silu_quant.cu:22-69: r = RN_T( float(silu_h(g)) * float(u) ) (the __hmul product of two fp16 values is
 * one correctly rounded multiply; the float product of two 11-bit significands is exact), absmax over the row of r,
 * inverse = absmax > 0 ? 127 / absmax : 0, scale = absmax / 127, q = q8(float(r) * inverse).
 * gu: [M, 2I] (gate = columns 0..I-1, up = I..2I-1); q: [M, I]; s: [M].  The bf16 variant (dtype 1) is the same
 * chain in bf16, as vLLM's silu_and_mul computes it for bf16 models (the reference kernel is fp16 only).
 * ------------------------------------------------------------------------------------------------------------------ */
void o_silu_mul_quant(const uint16_t* gu, int dtype, long M, long I, int8_t* q, float* s, uint16_t* act) {
    for (long m = 0; m < M; ++m) {
        const uint16_t* g = gu + m * 2 * I;
        const uint16_t* u = g + I;
        uint16_t* r = act + m * I;
        float amax = 0.0f;
        for (long i = 0; i < I; ++i) {
            const float sg = to_f(o_silu_h(g[i], dtype), dtype);
            r[i] = from_f(sg * to_f(u[i], dtype), dtype);
            const float v = fabsf(to_f(r[i], dtype));
            if (v > amax) amax = v;
        }
        const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        s[m] = amax / 127.0f;
        for (long i = 0; i < I; ++i) q[m * I + i] = q8(to_f(r[i], dtype) * inv);
    }
}

/* ------------------------------------------------------------------------------------------------------------------
 * Fused residual add + RMSNorm + dynamic per-token int8 quantization: the producer of the gate_up input in the
 * reference's MLP tail, ops.rms_norm_dynamic_per_token_quant(h, w1, eps, torch.int8, None, res) at
 * vllm_turing/tailoverlap.py:145 (w1 = 1 + w precomputed for GemmaRMSNorm at :123).  The op is vLLM's (third-party,
 * not in the reference tree); restated from its published kernel, per row:
 *   s[k]  = float(x[k]) + float(r[k])                       (r absent: s = float(x))
 *   r[k]  = RN_T(s[k])                                      (the residual is updated in place)
 *   rms   = 1 / sqrt(mean(s^2) + eps)
 *   y[k]  = float( RN_T( float(RN_T(RN32(s[k] * rms))) * float(w[k]) ) )   (the 16-bit product is exact in float)
 *   scale = max(RN32(min(absmax(y), ub) / 127), FLT_EPSILON);  q[k] = clamp(rint(RN32(y[k] * RN32(1 / scale))))
 * vLLM sums s^2 in float32 in its block-reduction order and takes rsqrtf; this build's contract fixes both: the sum
 * is taken in float64 (each square exact, the sum order-free to ~1e-12) and rounded once, ms = RN32(ss / K), and
 * rms = RN32(1 / RN32(sqrt(RN32(ms + eps)))).  The unpinned residue against vLLM is therefore the last float32 bit of
 * rms, which moves a 16-bit y only when s * rms sits within ~1e-6 of a rounding boundary.
 * x: [M, K] bit patterns (row stride K); res: [M, K] or NULL, updated; w: [K]; ub: scale upper bound or NULL;
 * q: [M, K]; s: [M]; y (optional, may be NULL): the normalised 16-bit row, [M, K].
 * ------------------------------------------------------------------------------------------------------------------ */
void o_rms_norm_quant(const uint16_t* x, uint16_t* res, const uint16_t* w, const float* ub, float eps, long M, long K,
                      int dtype, int8_t* q, float* scales, uint16_t* y, float* sbuf) {
    /* sbuf: caller scratch of K floats (the row's s) */
    for (long m = 0; m < M; ++m) {
        const uint16_t* xr = x + m * K;
        uint16_t* rr = res ? res + m * K : 0;
        double ss = 0.0;
        for (long k = 0; k < K; ++k) {
            float v = to_f(xr[k], dtype);
            if (rr) {
                v = v + to_f(rr[k], dtype);
                rr[k] = from_f(v, dtype);
            }
            sbuf[k] = v;
            ss += (double)v * (double)v;                         /* exact square of a float in double */
        }
        const float ms = (float)(ss / (double)K);
        const float rms = 1.0f / sqrtf(ms + eps);
        float amax = 0.0f;
        for (long k = 0; k < K; ++k) {
            const float t = sbuf[k] * rms;
            const float p = to_f(from_f(t, dtype), dtype) * to_f(w[k], dtype);    /* exact */
            const uint16_t yb = from_f(p, dtype);
            if (y) y[m * K + k] = yb;
            const float yv = to_f(yb, dtype);
            sbuf[k] = yv;
            if (fabsf(yv) > amax) amax = fabsf(yv);
        }
        float a = amax;
        if (ub && *ub < a) a = *ub;
        float scale = a / 127.0f;
        if (!(scale >= FLT_EPSILON)) scale = FLT_EPSILON;
        scales[m] = scale;
        const float inv = 1.0f / scale;
        for (long k = 0; k < K; ++k) q[m * K + k] = q8(sbuf[k] * inv);
    }
}

/* ------------------------------------------------------------------------------------------------------------------
 * AR8: int8 with an fp16 scale per 128-element group, the compressed operand of the reference's large all-reduce
 * (csrc/host_ar.cu:133-201).  Per group: amax = max|float(x)|, scale = RN16(RN32(amax / 127)), s = float(scale),
 * inv = s > 0 ? RN32(1 / s) : 0, q = clamp(rint(RN32(float(x) * inv)), -127, 127) (the kernel clamps at -127, not
 * -128).  packed = n int8 then n / 128 fp16 scales.  x: n fp16 bit patterns, n % 128 == 0.
 * ------------------------------------------------------------------------------------------------------------------ */
void o_ar8_quant(const uint16_t* x, long n, uint8_t* packed) {
    int8_t* q = (int8_t*)packed;
    uint16_t* sc = (uint16_t*)(packed + n);
    for (long g = 0; g < n / 128; ++g) {
        float amax = 0.0f;
        for (int i = 0; i < 128; ++i) {
            const float v = fabsf(o_h2f(x[g * 128 + i]));
            if (v > amax) amax = v;
        }
        const uint16_t sh = o_f2h(amax / 127.0f);
        const float s = o_h2f(sh);
        const float inv = s > 0.0f ? 1.0f / s : 0.0f;
        for (int i = 0; i < 128; ++i) {
            float r = rintf(o_h2f(x[g * 128 + i]) * inv);
            if (r < -127.0f) r = -127.0f;
            if (r > 127.0f) r = 127.0f;
            q[g * 128 + i] = (int8_t)r;
        }
        sc[g] = sh;
    }
}

/* The sum over `ranks` packed blocks (rank order, each n + n / 64 bytes) of the dequantised values, rounded once to
 * fp16 (csrc/host_ar.cu:166-183 for two ranks: u * a0 + w * a1, both products exact in float32, one rounding).  For
 * more ranks the float32 sum runs in rank order, each step a fused multiply-add of an exact product (for two ranks
 * this is the reference's single rounding). */
void o_ar8_dequant_sum(const uint8_t* gathered, long n, int ranks, uint16_t* out) {
    const long m = n + n / 64;
    for (long i = 0; i < n; ++i) {
        const long g = i / 128;
        float acc = 0.0f;
        for (int r = 0; r < ranks; ++r) {
            const int8_t* q = (const int8_t*)(gathered + r * m);
            const uint16_t* sc = (const uint16_t*)(gathered + r * m + n);
            const float p = (float)q[i] * o_h2f(sc[g]);              /* exact: 8-bit x 11-bit significands */
            acc = r == 0 ? p : fmaf((float)q[i], o_h2f(sc[g]), acc);
            (void)p;
        }
        out[i] = o_f2h(acc);
    }
}

/* ------------------------------------------------------------------------------------------------------------------
 * The int8 LM head (W8A16), csrc/w8a16_gemv.cu:98-117: out[m, n] = RN_T( fmaf( acc, s[row], b ) ), acc the float32 sum
 * of float(w[row, k]) * float(x[m, k]) over k, b = float(bias[row]) or +0, row = rows ? rows[n] : n.  The reference
 * sums in its own lane order; here acc is the float64 sum (every product exact) rounded once to float32, the value any
 * summation order approximates.  x: [M, K] bit patterns of dtype; w: int8 [w_rows, K]; s: [w_rows]; out: [M, N].
 * ------------------------------------------------------------------------------------------------------------------ */
void o_w8a16(const uint16_t* x, const int8_t* w, const float* s, const uint16_t* bias, const int32_t* rows,
             uint16_t* out, long M, long N, long K, int dtype) {
    for (long m = 0; m < M; ++m) {
        for (long n = 0; n < N; ++n) {
            const long row = rows ? rows[n] : n;
            double acc = 0.0;
            for (long k = 0; k < K; ++k) acc += (double)w[row * K + k] * (double)to_f(x[m * K + k], dtype);
            const float b = bias ? to_f(bias[row], dtype) : 0.0f;
            out[m * N + n] = from_f(fmaf((float)acc, s[row], b), dtype);
        }
    }
}
