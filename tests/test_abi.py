"""CPU-only checks of the C ABI library and the host-side logic (no kernel is launched: no GPU here).

* libw8a8_mi355.so builds for gfx950 and exports every entry point include/w8a8_mi355.h declares;
* argument validation returns the documented codes before any HIP call;
* the dispatch predicates (vllm_turing/w8a8.py:38-46,58-66,78-79) select the reference's path for each M and layout;
* the product package never imports the oracle, and has no torch fallback for the matmul.
"""
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    txt = open(os.path.join(ROOT, "include", "w8a8_mi355.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return re.findall(r"^\s*(?:int|long)\s+(\w+)\s*\(", txt, flags=re.M)


@pytest.fixture(scope="module")
def L():
    from vllm_turing_amd import _lib
    return _lib.lib()


def test_header_and_signatures_agree():
    from vllm_turing_amd import _lib
    syms = header_symbols()
    assert sorted(syms) == sorted(_lib.SIGNATURES)


def test_library_exports_every_symbol(L):
    for s in header_symbols():
        assert hasattr(L, s), s


def test_library_is_gfx950_only():
    from vllm_turing_amd import _build
    so = _build.so_path()
    data = open(so, "rb").read()
    assert b"gfx950" in data
    assert b"gfx942" not in data and b"gfx90a" not in data


def test_argument_validation_codes(L):
    # w8a8_gemv / w8a8_mma: -1 for M out of range or K % 16 (csrc/w8a8_gemv.cu:349-351, :332-334)
    assert L.w8a8_gemv(16, 16, 0, 0, None, 0, 0, 64, 64, 1, 1, 0, None) == -1
    assert L.w8a8_gemv(16, 16, 0, 0, None, 0, 17, 64, 64, 1, 1, 0, None) == -1
    assert L.w8a8_gemv(16, 16, 0, 0, None, 0, 4, 64, 40, 1, 1, 0, None) == -1
    assert L.w8a8_mma(16, 16, 0, 0, None, 0, 33, 64, 64, 1, 1, 0, None) == -1
    assert L.w8a8_gemv(17, 16, 0, 0, None, 0, 4, 64, 64, 1, 1, 0, None) == -1     # misaligned a
    assert L.w8a8_gemv(16, 16, 0, 0, None, 0, 4, 64, 64, 1, 1, 2, None) == -1     # bad dtype
    # w8a8_big: 1 = cannot implement (csrc/w8a8_big.cu:57)
    assert L.w8a8_big(16, 16, 0, 0, 0, 64, 24, 64, 0, None) == 1                  # N % 16
    assert L.w8a8_big(16, 16, 0, 0, 0, 64, 64, 72, 0, None) == 1                  # K % 16
    assert L.w8a8_scaled_mm(16, 16, 0, 0, None, 0, 0, 64, 64, 1, 1, 0, None) == -1
    # w8a8_scaled_mm_ws: a shape that splits needs its workspace (missing, too small, misaligned: -1)
    need = L.w8a8_scaled_mm_ws_size(512, 12288, 5120)
    assert need > 4096 and (need - 4096) % (256 * 1024) == 0
    assert L.w8a8_scaled_mm_ws(16, 16, 0, 0, None, 0, 512, 12288, 5120, 1, 1, 1, None, 0, None) == -1
    assert L.w8a8_scaled_mm_ws(16, 16, 0, 0, None, 0, 512, 12288, 5120, 1, 1, 1, 4096, need - 1, None) == -1
    assert L.w8a8_scaled_mm_ws(16, 16, 0, 0, None, 0, 512, 12288, 5120, 1, 1, 1, 4100, need, None) == -1
    assert L.w8a8_scaled_mm_ws(16, 16, 0, 0, None, 0, 0, 64, 64, 1, 1, 0, None, 0, None) == -1
    assert L.w8a8_scaled_mm_ws(16, 16, 0, 0, None, 0, 64, 64, 64, 1, 1, 3, None, 0, None) == -1   # dtype 0..2
    assert L.w8a8_scaled_mm_ws_size(0, 64, 64) == -1 and L.w8a8_scaled_mm_ws_size(64, 64, 8) == -1
    assert L.w8a8_scaled_mm_ws_size(200, 1024, 5120) == 0       # a mid-M shape: no split
    assert L.w8a8_scaled_mm_ws_size(4096, 12288, 5120) == 0     # 768 super tiles: whole rounds on 256 CUs
    assert L.w8a8_scaled_mm_ws_size(512, 12288, 512) == 0       # 4 K stages: pieces would be under 4 stages
    # 64-row tiles over more than 12288 weight rows: two K pieces where they fit two per CU (256 CUs), 16 KB each
    assert L.w8a8_scaled_mm_ws_size(64, 16384, 5120) == 4096 + 256 * 2 * 16384
    assert L.w8a8_scaled_mm_ws_size(33, 17408, 5120) == 4096 + 272 * 2 * 16384
    assert L.w8a8_scaled_mm_ws_size(64, 20480, 5120) == 4096 + 320 * 2 * 16384     # 5/4 tiles per CU
    assert L.w8a8_scaled_mm_ws_size(64, 20544, 5120) == 0       # 321 tiles: past 5/4 per CU
    assert L.w8a8_scaled_mm_ws_size(64, 24576, 5120) == 0       # 384 tiles
    assert L.w8a8_scaled_mm_ws_size(96, 13312, 5120) == 0       # two tile rows: 416 tiles
    assert L.w8a8_scaled_mm_ws_size(64, 16384, 2048) == 0       # 16 stages: pieces of 8
    assert L.w8a8_scaled_mm_ws_size(32, 16384, 5120) == 0       # 32 rows run on the streaming kernel
    # at most 12288 weight rows: as many pieces as fill two workgroups per CU, where N > 4096 or K >= 64 stages
    assert L.w8a8_scaled_mm_ws_size(64, 12288, 5120) == 4096 + 192 * 2 * 16384
    assert L.w8a8_scaled_mm_ws_size(128, 5120, 17408) == 4096 + 160 * 3 * 16384
    assert L.w8a8_scaled_mm_ws_size(64, 1024, 17408) == 4096 + 16 * 8 * 16384
    assert L.w8a8_scaled_mm_ws_size(64, 4096, 5120) == 0        # 40 stages, N <= 4096
    assert L.w8a8_scaled_mm_ws_size(128, 12288, 5120) == 0      # 384 tiles: one piece each
    assert L.w8a8_scaled_mm_ws_size(192, 5120, 17408) == 4096 + 240 * 2 * 16384     # 129..256 rows, K >= 64 stages
    assert L.w8a8_scaled_mm_ws_size(256, 5120, 5120) == 0       # 129..256 rows at 40 stages
    assert L.w8a8_scaled_mm_ws_size(256, 5120, 17408) == 0      # 320 tiles: one piece each
    # w8a8_gemv_silu: -1 on bad arguments, 1 where the VALU GEMV does not take M or K
    assert L.w8a8_gemv_silu(16, 16, 0, 0, None, 16, 1, 0, 5120, 1, 1, 0, None) == -1      # I < 1
    assert L.w8a8_gemv_silu(16, 16, 0, 0, None, 16, 1, 64, 40, 1, 1, 0, None) == -1      # K % 16
    assert L.w8a8_gemv_silu(16, 16, 0, 0, None, None, 1, 64, 64, 1, 1, 0, None) == -1    # no output
    assert L.w8a8_gemv_silu(16, 16, 0, 0, None, 16, 6, 64, 64, 1, 1, 0, None) == 1       # M = 6: not the VALU GEMV
    assert L.w8a8_gemv_silu(16, 16, 0, 0, None, 16, 4, 64, 8192, 1, 1, 0, None) == 1     # K past four rows' limit
    # w8a8_scaled_mm_noalloc: the same validation, before any HIP call
    assert L.w8a8_scaled_mm_noalloc(16, 16, 0, 0, None, 0, 0, 64, 64, 1, 1, 0, None) == -1
    assert L.w8a8_scaled_mm_noalloc(16, 16, 0, 0, None, 0, 64, 64, 40, 1, 1, 0, None) == -1   # K % 16
    assert L.w8a8_scaled_mm_noalloc(17, 16, 0, 0, None, 0, 64, 64, 64, 1, 1, 0, None) == -1   # misaligned a
    assert L.w8a8_scaled_mm_noalloc(16, 16, 0, 0, None, 0, 64, 64, 64, 1, 1, 3, None) == -1   # dtype 0..2
    assert L.w8a8_i32(16, 16, 0, 65, 64, 64, 0, None) == -1                       # streaming kernel: M <= 64
    assert L.w8a8_i32(16, 16, 0, 6, 64, 64, 2, None) == -1                       # VALU kernel: M <= 5
    assert L.w8a8_i32(16, 16, 0, 1, 64, 17424, 2, None) == -1                    # K <= 17408 at one row
    assert L.w8a8_i32(16, 16, 0, 2, 64, 8208, 2, None) == -1                     # K <= 8192 at two rows
    assert L.w8a8_i32(16, 16, 0, 4, 64, 5136, 2, None) == -1                     # K <= 5120 at four rows
    assert L.w8a8_i32(16, 16, 0, 4, 64, 64, 6, None) == -1
    assert L.w8a8_i32(16, 16, 0, 40, 64, 131072, 1, None) == -1                 # K < 131072: exact int32 sums
    assert L.w8a8_scaled_mm(16, 16, 0, 0, None, 0, 40, 64, 131072, 1, 1, 0, None) == -1
    # silu_mul_quant: 1 = bad I, 0 for M == 0 (csrc/silu_quant.cu:72-73)
    assert L.silu_mul_quant(None, None, None, 4, 12, None) == 1
    assert L.silu_mul_quant(None, None, None, 0, 16, None) == 0
    assert L.silu_mul_quant_bf16(None, None, None, 4, 65544, None) == 1
    assert L.per_token_quant(None, None, None, 4, 16, 16, 0, None) == -1
    assert L.per_token_quant(16, 16, 16, 0, 16, 16, 0, None) == 0
    assert L.silu_table(None, 0, None) == -1
    assert L.silu_mul_quant_path(16, 16, 16, 4, 16, 2, 1, None) == 1            # dtype
    assert L.silu_mul_quant_path(16, 16, 16, 4, 16, 0, 0, None) == 1            # path 1 or 2
    assert L.silu_mul_quant_path(16, 16, 16, 4, 12, 0, 1, None) == 1            # I % 8
    assert L.w8a16_gemv(16, 16, 16, None, 16, 33, 64, 64, 0, None) == -1        # M <= 32
    assert L.w8a16_gemv(16, 16, 16, None, 16, 4, 64, 72, 0, None) == -1         # K % 16
    assert L.w8a16_gemv(16, 16, 16, None, 16, 4, 64, 64, 2, None) == -1         # dtype
    # the reference's 11-argument gathered entry (csrc/w8a16_gemv.cu:145-147): rows = NULL means all rows
    assert L.w8a16_gemv_rows(16, 16, 16, None, 16, 33, 64, 64, 0, None, None) == -1     # M <= 32
    assert L.w8a16_gemv_rows(16, 16, 16, None, 16, 4, 64, 72, 0, 16, None) == -1       # K % 16
    assert L.w8a16_gemv_rows_bounded(16, 16, 16, None, 16, 4, 64, 64, 0, None, 64, None) == -1   # rows required
    assert L.w8a16_gemv_rows_bounded(16, 16, 16, None, 16, 4, 64, 64, 0, 16, 0, None) == -1      # w_rows >= 1
    # w8a16_mma (csrc/w8a16_mma.cu:176-191): -1 for M outside 1..64, odd N, K not a multiple of cfg's k-tile;
    # -2 for the 512-byte k-tile above 32 rows
    assert L.w8a16_mma(16, 16, 16, None, 16, 0, 64, 512, 2, None) == -1
    assert L.w8a16_mma(16, 16, 16, None, 16, 65, 64, 512, 1, None) == -1
    assert L.w8a16_mma(16, 16, 16, None, 16, 8, 63, 512, 2, None) == -1
    assert L.w8a16_mma(16, 16, 16, None, 16, 8, 64, 384, 2, None) == -1            # 512-byte k-tile
    assert L.w8a16_mma(16, 16, 16, None, 16, 8, 64, 320, 1, None) == -1            # 256-byte k-tile
    assert L.w8a16_mma(16, 16, 16, None, 16, 8, 64, 192, 0, None) == -1            # 128-byte k-tile
    assert L.w8a16_mma(16, 16, 16, None, 16, 33, 64, 5120, 2, None) == -2
    assert L.w8a16_mma(8, 16, 16, None, 16, 8, 64, 512, 2, None) == -1             # x 16-byte aligned
    assert L.w8a16_mma(None, 16, 16, None, 16, 8, 64, 512, 2, None) == -1
    assert L.w8a8_gemv_quant(16, 64, 16, 16, 16, 16, None, 16, 17, 64, 64, 1, 0, None) == -1     # M <= 16
    assert L.w8a8_gemv_quant(16, 32, 16, 16, 16, 16, None, 16, 4, 64, 64, 1, 0, None) == -1      # ldx >= K
    assert L.w8a8_gemv_quant(None, 64, 16, 16, 16, 16, None, 16, 4, 64, 64, 1, 0, None) == -1    # x
    assert L.w8a8_gemv_quant(16, 64, 16, 16, 16, 16, None, 16, 4, 64, 72, 1, 0, None) == -1      # K % 16
    assert L.w8a8_gemv_quant(16, 64, 8, 16, 16, 16, None, 16, 4, 64, 64, 1, 0, None) == -1       # xq aligned
    assert L.hbm_read(None, 4, 1024, 16, None) == -1
    assert L.hbm_read(16, 4, 1000, 16, None) == -1                                 # K % 16
    assert L.hbm_read(16, 4, 17424, 16, None) == -1                                # K <= 17408
    assert L.hbm_read(8, 4, 1024, 16, None) == -1                                  # 16-byte aligned
    assert L.silu_table(16, 4, None) == -1                                         # 0..3
    assert L.ar8_quant(16, 16, 100, None) == -1                                 # n % 128
    assert L.ar8_quant(8, 16, 128, None) == -1                                  # x 16-byte aligned
    assert L.ar8_quant(16, 16, 0, None) == 0
    assert L.ar8_dequant_sum_ranks(16, 16, 128, 9, None) == -1                  # 1..8 ranks
    assert L.ar8_dequant_sum(16, 16, 130, None) == -1
    assert L.f32_to_16(None, None, 4, 1, None) == -1
    assert L.f32_to_16(16, 16, 4, 2, None) == -1
    assert L.f32_to_16(16, 16, 0, 1, None) == 0


def _t(M, N, K, bias=False, per_tensor=False, out_dtype=torch.float16):
    a = torch.zeros(M, K, dtype=torch.int8)
    w = torch.zeros(N, K, dtype=torch.int8)
    sa = torch.ones(1 if per_tensor else M, 1)
    sb = torch.ones(N, 1)
    out = torch.empty(M, N, dtype=out_dtype)
    return out, a, w.t(), sa, sb, (torch.zeros(N, dtype=out_dtype) if bias else None)


def path(*args):
    from vllm_turing_amd import w8a8
    if w8a8.gemv_ok(*args):
        return "gemv"
    if w8a8.mma_ok(*args):
        return "mma"
    if w8a8.big_ok(*args):
        return "big"
    return "general"


@pytest.mark.parametrize("M,kw,want", [
    (1, {}, "gemv"), (12, {}, "gemv"), (13, {}, "mma"), (32, {}, "mma"), (33, {}, "big"), (4096, {}, "big"),
    (8, {"bias": True}, "gemv"), (20, {"per_tensor": True}, "mma"), (64, {"bias": True}, "general"),
    (64, {"per_tensor": True}, "general"), (4, {"out_dtype": torch.float32}, "general"),
])
def test_dispatch_truth_table(M, kw, want):
    assert path(*_t(M, 256, 512, **kw)) == want


def test_dispatch_layout_rejections():
    out, a, b, sa, sb, bias = _t(4, 256, 512)
    assert path(out, a, b.contiguous(), sa, sb, bias) == "general"        # b not the stride-(1, K) view
    assert path(out, a[:, :500], b[:500], sa, sb, bias) == "general"      # K % 16
    out, a, b, sa, sb, bias = _t(40, 250, 512)
    assert path(out, a, b, sa, sb, bias) == "general"                     # big needs N % 16


def test_product_does_not_use_the_oracle():
    pkg = os.path.join(ROOT, "vllm_turing_amd")
    for dp, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h")):
                src = open(os.path.join(dp, f)).read()
                assert "import oracle" not in src and "from oracle" not in src and "liboracle" not in src, f
                assert "_int_mm" not in src, f                              # no torch matmul fallback
