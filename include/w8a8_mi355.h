/*
 * C ABI of the MI355X (gfx950) W8A8 SmoothQuant linear path: libw8a8_mi355.so.
 *
 * Plain pointers and sizes only.  Every buffer is allocated by the caller (torch tensors on the Python side); no entry
 * point allocates or synchronizes, so every launch is asynchronous on `stream` (a hipStream_t, e.g.
 * torch.cuda.current_stream().cuda_stream) and can be captured in a HIP graph.  None keeps state, except in the
 * workspace a caller passes to w8a8_scaled_mm_ws and in the per-GPU scratch of w8a8_scaled_mm_noalloc (tile counters
 * that every call leaves at zero).  Argument validation happens before any HIP call and returns the documented code.
 *
 * dtype: 0 = float16, 1 = bfloat16 (activations, bias and output).  Weights are int8 [N, K] row-major (the layout vLLM
 * stores; its cutlass_scaled_mm receives the [K, N] stride-(1, K) view of it).  Scales are float32: sa [M] (sa_rows=1)
 * or [1] (per-tensor), sw [N] (sw_rows=1) or [1].  All int8 operands must be 16-byte aligned with K % 16 == 0.
 */
#ifndef W8A8_MI355_H
#define W8A8_MI355_H

#ifdef __cplusplus
extern "C" {
#endif

/* Small-M W8A8 GEMV, M in [1, 16]: out[m, n] = T(fma(float(acc) * sa[m], sw[n], bias[n] or 0)).
 * Replaces vllm_turing/csrc/w8a8_gemv.cu:347 (same arguments).  Returns -1 on bad arguments, else the HIP error code
 * of the launch (0 = success). */
int w8a8_gemv(const void* a, const void* w, const void* sa, const void* sw, const void* bias, void* out, int M, int N,
              int K, int sa_rows, int sw_rows, int dtype, void* stream);

/* Small-M W8A8 GEMM, M in [1, 32], same arithmetic as w8a8_gemv.
 * Replaces vllm_turing/csrc/w8a8_gemv.cu:330 (same arguments and return codes). */
int w8a8_mma(const void* a, const void* w, const void* sa, const void* sw, const void* bias, void* out, int M, int N,
             int K, int sa_rows, int sw_rows, int dtype, void* stream);

/* The small-M W8A8 GEMV from 16-bit activations, quantization fused: x [M, K] fp16 (dtype 0) / bf16 (dtype 1) with
 * row stride ldx elements is quantized per token exactly as per_token_quant does (its int8 rows and float32 scales are
 * written to xq [M, K] and xs [M]) and multiplied as w8a8_gemv does (small-M epilogue, sa = xs), M in [1, 16]; out
 * [M, N] in the same dtype.  At one row (K <= 17408, x 16-byte aligned, ldx % 8 == 0) each workgroup quantizes the
 * row itself, so no separate quantization launch runs (the decode o_proj / out_proj input); otherwise the two steps
 * run as two launches.  No counterpart in the reference, whose
 * quantization is fused into the producer by inductor (vllm_turing/quantfuse.py:1-10).  Returns -1 on bad arguments,
 * else the HIP launch error. */
int w8a8_gemv_quant(const void* x, long ldx, void* xq, void* xs, const void* w, const void* sw, const void* bias,
                    void* out, int M, int N, int K, int sw_rows, int dtype, void* stream);

/* The decode MLP's gate_up GEMV with SiLU * up in its epilogue: a [M, K] int8, w [2I, K] int8 (gate rows 0..I-1, up
 * rows I..2I-1), sa [M] or [1], sw [2I] or [1], bias [2I] of the output type or null; h [M, I] = T(float(silu_h(g)) *
 * float(u)) where g = out[m, p] and u = out[m, p + I] are the outputs w8a8_gemv would write (small-M epilogue) and
 * silu_h is silu_mul_quant's 16-bit silu, so per_token_quant(h) equals silu_mul_quant(w8a8_gemv output) bit for bit.
 * Taken where the VALU GEMV takes M and K (M <= 5; K <= 17408 at one row, 8192 at two or three, 5120 at four or
 * five).  No counterpart in the reference, whose MLP runs the GEMV and silu_quant.cu:71 as two launches
 * (vllm_turing/tailoverlap.py:146-151).  Returns -1 on bad arguments, 1 for M or K outside that range, else the HIP
 * launch error. */
int w8a8_gemv_silu(const void* a, const void* w, const void* sa, const void* sw, const void* bias, void* h, int M,
                   int I, int K, int sa_rows, int sw_rows, int dtype, void* stream);

/* Prefill W8A8 GEMM, any M (dispatched for M > 32), per-row sa [M] and per-column sw [N], no bias, N % 16 == 0:
 * out[m, n] = T(sa[m] * float(float(acc) * sw[n])).
 * Replaces vllm_turing/csrc/w8a8_big.cu:66 (same arguments).  Returns 0 ok, 1 cannot implement (shape, alignment),
 * 3 launch failed. */
int w8a8_big(const void* A, const void* W, const void* sa, const void* sw, void* out, int M, int N, int K, int dtype,
             void* stream);

/* General scaled int8 matmul, any M, optional bias, per-row or per-tensor scales, with the large-M epilogue
 * out = T(sa * float(float(acc) * sw)) or, with a bias, T(fma(sa, float(float(acc) * sw), bias)).
 * Replaces the vLLM torch.ops._C.cutlass_scaled_mm fallback the reference calls at vllm_turing/w8a8.py:117 (same
 * operands as w8a8_gemv).  Returns -1 on bad arguments, else the HIP error code of the launch. */
int w8a8_scaled_mm(const void* a, const void* w, const void* sa, const void* sw, const void* bias, void* out, int M,
                   int N, int K, int sa_rows, int sw_rows, int dtype, void* stream);

/* w8a8_scaled_mm (and so w8a8_big, which is its no-bias per-row / per-column case) with a caller workspace for the
 * prefill GEMM's K splits: when the 256 x 256 super tiles leave a last partial round of at most half the CUs, each of
 * those tiles runs as 2..8 K pieces (at least 3 after whole rounds), and 33..128 rows run their 64 x 64 tiles as K
 * pieces of at least 16 stages: against more than 12288 weight rows 2 pieces where the tiles number at most 5/4 of
 * the CUs (up to 20480 weight rows at 64 rows on 256 CUs; past one tile per CU some tiles' pieces are of unequal
 * length), against fewer (more than 4096, or K of at least 8192) as many as fill two workgroups per CU, as do
 * 129..256 rows against at most 8192 weight rows with K of at least 8192; the pieces' int32 partial sums meet in the
 * workspace (the last piece to finish adds them and runs the epilogue; the results are bit-identical to
 * w8a8_scaled_mm's).  workspace: 16-byte aligned, ws_bytes >= w8a8_scaled_mm_ws_size(M, N, K) (it may be null when
 * that is 0); its first 4 KB (tile counters) must be zero before the first call, and every call leaves them zero.
 * Calls that share a workspace must not overlap.
 * dtype 2 writes the raw int32 accumulators acc [M, N] to out (sa, sw, bias unused; for checking).  Returns -1 on bad
 * arguments (a missing or too small workspace included), else the HIP error code of the launches.
 * No counterpart in the reference, whose w8a8_big rejects a workspace (vllm_turing/csrc/w8a8_big.cu:57-59); this
 * serves the same callers as w8a8_big and w8a8_scaled_mm (vllm_turing/w8a8.py:92-101,117). */
int w8a8_scaled_mm_ws(const void* a, const void* w, const void* sa, const void* sw, const void* bias, void* out,
                      int M, int N, int K, int sa_rows, int sw_rows, int dtype, void* workspace, long ws_bytes,
                      void* stream);

/* Workspace bytes w8a8_scaled_mm_ws takes for M x N x K on the current device: 0 when the shape does not split, at
 * most 4 KB + 256 KB per CU; -1 for M, N < 1 or K < 16. */
long w8a8_scaled_mm_ws_size(int M, int N, int K);

/* w8a8_scaled_mm_ws that allocates nothing: the same arguments without the workspace, whose place the library's own
 * scratch takes (a static device array of 64 MiB + 4 KiB per GPU, held until the process ends; its address is looked
 * up once per device).  No counterpart in the reference: for callers that cannot allocate (code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc).  Every call on a GPU shares that GPU's scratch, so
 * calls that overlap on one GPU (other streams or threads) race.  Returns -1 on bad arguments, -2 when the shape's K
 * split needs more than the scratch holds (more than 256 CUs), -3 when the scratch's address cannot be had, else the
 * HIP error code of the launches. */
int w8a8_scaled_mm_noalloc(const void* a, const void* w, const void* sa, const void* sw, const void* bias, void* out,
                           int M, int N, int K, int sa_rows, int sw_rows, int dtype, void* stream);

/* Dynamic symmetric per-token int8 quantization: scales[m] = absmax_m / 127,
 * q[m, k] = clamp(rint(float(x[m, k]) * (127 / absmax_m)), -128, 127); a zero row gives q = 0 and scale 0.
 * x: [M, K] fp16/bf16 with row stride ldx elements; q: [M, K] int8 contiguous; scales: [M] float32.
 * Replaces the eager vllm._custom_ops.scaled_int8_quant(input, None, None, True) that
 * vllm_turing/quantfuse.py:35-39 leaves to vLLM.  Returns 0, -1 on bad arguments, or the HIP launch error. */
int per_token_quant(const void* x, void* q, void* scales, int M, int K, long ldx, int dtype, void* stream);

/* SiLU(gate) * up + per-row dynamic int8 quantization, fp16: gu [M, 2I] (gate = columns [0, I), up = [I, 2I)),
 * q [M, I] int8, scales [M] float32.  I % 8 == 0, I <= 65536.
 * Replaces vllm_turing/csrc/silu_quant.cu:71 (same arguments).  Returns 0 ok, 1 bad I, 2 launch error. */
int silu_mul_quant(const void* gu, void* q, void* scales, int M, int I, void* stream);

/* The same for bfloat16 activations.  No counterpart in the reference (its kernel is fp16 only); same codes. */
int silu_mul_quant_bf16(const void* gu, void* q, void* scales, int M, int I, void* stream);

/* Residual add + RMSNorm + dynamic per-token int8 quantization: vLLM's rms_norm_dynamic_per_token_quant(input, weight,
 * epsilon, torch.int8, scale_ub, residual), the producer of the gate_up input in the reference's MLP tail
 * (vllm_turing/tailoverlap.py:145; the GemmaRMSNorm weight 1 + w is precomputed by the caller, :123).  x: [M, K]
 * fp16 (dtype 0) or bf16 (dtype 1) row-major; residual: [M, K] of the same type, updated in place to RN(x + residual),
 * or NULL; weight: [K]; scale_ub: one float32 bound on the row absmax, or NULL; q: [M, K] int8; scales: [M] float32.
 * Returns 0, -1 on bad arguments, else the HIP launch error. */
int rms_norm_quant(const void* x, void* residual, const void* weight, const void* scale_ub, float eps, void* q,
                   void* scales, int M, int K, int dtype, void* stream);

/* AR8 group quantization, the compressed operand of the reference's large all-reduce (csrc/host_ar.cu:186-192, same
 * arguments): x n fp16 (n % 128 == 0) -> packed = n int8 then n / 128 fp16 scales (scale = RN16(absmax / 127) per
 * 128 values, q = clamp(rint(x / scale), -127, 127)).  Returns 0, -1 on bad arguments, else the HIP launch error. */
int ar8_quant(const void* x, void* packed, int n, void* stream);

/* The sum of two ranks' dequantised AR8 blocks (csrc/host_ar.cu:194-201, same arguments): gathered = two packed
 * blocks in rank order (n + n / 64 bytes each) -> out n fp16.  Returns 0, -1 on bad arguments, else the HIP error. */
int ar8_dequant_sum(const void* gathered, void* out, int n, void* stream);

/* The same for 1..8 ranks in rank order (no counterpart in the reference, which is two-rank only; for the 8 GPUs of
 * an xGMI node). */
int ar8_dequant_sum_ranks(const void* gathered, void* out, int n, int ranks, void* stream);

/* The int8 LM head, W8A16 (csrc/w8a16_gemv.cu:145-154, same arguments): out [M, N] = x [M, K] (fp16 dtype 0 / bf16
 * dtype 1) times the int8 rows w [N, K] with float32 per-row scales s [N] and an optional bias [N] of the activation
 * type: RN(fma(sum_k w x, s, bias)) with float32 sums.  M in 1..32 (the reference: 1..16), K % 16 == 0.  Returns -1 on
 * bad arguments, else the HIP launch error. */
int w8a16_gemv(const void* x, const void* w, const void* s, const void* bias, void* out, int M, int N, int K, int dtype,
               void* stream);

/* The same over the gathered weight rows rows[0..N) (int32 indexes into w; out is compact), for a pruned draft
 * vocabulary; rows = NULL computes all N rows.  Replaces vllm_turing/csrc/w8a16_gemv.cu:145-146 (same 11 arguments,
 * bound by vllm_turing/draftvocab.py:269 and tests/test_dhead.py:83).  As there, every index must name a row of w. */
int w8a16_gemv_rows(const void* x, const void* w, const void* s, const void* bias, void* out, int M, int N, int K,
                    int dtype, const void* rows, void* stream);

/* The gathered form with w's row count w_rows: indices are clamped to [0, w_rows) so the loads stay inside w.  No
 * counterpart in the reference (its indices are trusted).  Returns -1 on bad arguments or a null rows. */
int w8a16_gemv_rows_bounded(const void* x, const void* w, const void* s, const void* bias, void* out, int M, int N,
                            int K, int dtype, const void* rows, int w_rows, void* stream);

/* The int8 LM head for 5..64 rows with fp16 activations, the reference's tensor-core entry (vllm_turing/csrc/
 * w8a16_mma.cu:176-191, same arguments, bound by vllm_turing/lmhead.py:33-37,77): out [M, N] fp16 = x [M, K] fp16
 * times w [N, K] int8 with scales s [N] and bias [N] fp16 or NULL, float32 sums.  Returns -1 for M outside 1..64, an
 * odd N, or K not a multiple of cfg's k-tile (cfg 0: 128, 1: 256, other: 512 bytes); -2 for the 512-byte k-tile with
 * M > 32 (the reference's shared-memory limit); -1 on null or misaligned x / w; else the launch error.  Every cfg runs
 * the same kernel, so outputs do not depend on cfg. */
int w8a16_mma(const void* x, const void* w, const void* s, const void* bias, void* out, int M, int N, int K, int cfg,
              void* stream);

/* Test export: the raw int32 accumulators acc [M, N] = a . w^T of one kernel's main loop, for bit-exact accumulator
 * checks: kernel 0 the small-M MFMA streaming kernel (M <= 64), 1 the prefill kernel as dispatched, 2 the v_dot4
 * streaming kernel (M = 1 and K <= 17408, M = 2, 3 and K <= 8192, M = 4, 5 and K <= 5120), 3 and 4 the prefill
 * kernel's quarter-tile and full-tile (single-role wavefronts) configurations alone, 5 the full-tile configuration
 * with alternating wavefront groups alone.  No counterpart in the reference.  Returns -1 on bad arguments, else the
 * HIP launch error. */
int w8a8_i32(const void* a, const void* w, void* acc, int M, int N, int K, int kernel, void* stream);

/* Test export: silu_mul_quant (dtype 0) / silu_mul_quant_bf16 (dtype 1) through one of its two kernels, path 1 the
 * direct kernel (float32 exp and division per element), path 2 the table kernel (the device's 16-bit silu of every
 * gate pattern, built once per device, looked up in LDS), so that tests can compare them.  No counterpart in the
 * reference.  Returns silu_mul_quant's codes, and 1 where the table kernel does not apply (I > 40960, or its table
 * not yet built while the stream is being captured). */
int silu_mul_quant_path(const void* gu, void* q, void* scales, int M, int I, int dtype, int path, void* stream);

/* Test export: the device silu of all 65,536 input patterns of dtype, out[65536] uint16 bit patterns.  No
 * counterpart in the reference.  Returns -1 on bad arguments, else the HIP launch error. */
int silu_table(void* out, int dtype, void* stream);

/* Test export: out[i] (uint16 bit patterns) = the device's round-to-nearest-even of float32 x[i] to fp16 (dtype 0)
 * or bf16 (dtype 1), the rounding every 16-bit output of this library goes through.  No counterpart in the
 * reference.  Returns -1 on bad arguments, else the HIP launch error. */
int f32_to_16(const void* x, void* out, long n, int dtype, void* stream);

/* Test export: the M = 1 decode GEMV's weight stream without its math: rows x K bytes of src (16-byte aligned,
 * K % 16 == 0, K <= 17408) read exactly as w8a8_gemv reads its weights at one activation row (one-wavefront
 * workgroups of three rows, 1 KB per wavefront instruction, non-temporal loads, the next row's loads in flight) and
 * discarded: the read rate the GEMV is measured against.  sink: one int of device memory, written only if the XOR of
 * all words read equals 0x5a3c96e1.  No counterpart in the reference.  Returns -1 on bad arguments, else the launch
 * error. */
int hbm_read(const void* src, int rows, int K, void* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* W8A8_MI355_H */
