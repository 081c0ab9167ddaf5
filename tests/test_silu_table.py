"""The SiLU lookup tables generated at build time (vllm_turing_amd/silu_table.py) against the oracle's silu, which
is pinned to a 60-digit decimal exp in test_oracle_pins.py: all 65,536 fp16 and all 65,536 bf16 patterns, NaN where
the oracle gives NaN, known values, and the include file the build compiles in."""
import numpy as np
import pytest
import torch

from vllm_turing_amd import silu_table as gen


def _isnan(bits, dt):
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.float16 if dt == 0 else torch.bfloat16)
    return t.isnan().numpy()


@pytest.mark.parametrize("dt", [0, 1])
def test_table_matches_oracle(oracle_lib, dt):
    got = gen.values(dt)
    ref = oracle_lib.silu_table(dt)
    nan_g, nan_r = _isnan(got, dt), _isnan(ref, dt)
    assert np.array_equal(nan_g, nan_r)
    bad = np.nonzero((got != ref) & ~nan_r)[0]
    assert bad.size == 0, f"{bad.size} differ, first patterns {bad[:8]}"


def test_known_values():
    f16 = lambda v: int(np.array(v, np.float16).view(np.uint16))
    t = gen.values(0)
    assert t[f16(0.0)] == 0
    assert t[f16(1.0)] == f16(0.7310585786300049)
    assert t[f16(-1.0)] == f16(-0.2689414213699951)
    assert t[f16(20.0)] == f16(20.0)
    assert t[0x7C00] == 0x7C00                      # silu(+inf) = inf
    assert _isnan(t[np.array([0xFC00])], 0)[0]      # silu(-inf) = -inf / inf = NaN


def test_bf16_rounding_ties_to_even():
    vals = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 3.0e38, 1e-40], np.float32)
    got = gen.round16(vals, 1)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


def test_include_file(tmp_path):
    p = tmp_path / "silu_table.inc"
    gen.write_include(str(p))
    body = p.read_text().split("\n", 1)[1]
    nums = [int(x, 16) for x in body.replace("{", " ").replace("}", " ").replace(",", " ").split()]
    assert len(nums) == 2 * 65536
    assert np.array_equal(np.array(nums[:65536], np.uint16), gen.values(0))
    assert np.array_equal(np.array(nums[65536:], np.uint16), gen.values(1))
