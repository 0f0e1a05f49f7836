"""The no-allocation decode (llmtie_attn_decode_f16_noalloc) against the
scratch-taking one (llmtie_attn_decode_f16) it is a variant of: the same
kernels and plan, so the same bits, on two calls in a row (the second
smaller, so the fixed scratch holds the first call's leftovers), and a call
too large for the fixed scratch refused by name before any launch."""
import numpy as np
import pytest
import torch

import oracle
from tests.util import down, up, up_f16

pytestmark = pytest.mark.gpu


def _case(heads, kv, hd, cap, salt):
    return (up(oracle.seq(heads * hd, salt)), up_f16(oracle.seq(kv * cap * hd, salt + 1)),
            up_f16(oracle.seq(kv * cap * hd, salt + 2)))


def test_noalloc_decode_is_the_scratch_decode(gpu):
    from ttsxabe_amd.gpu import DecodeScratch
    for heads, kv, hd, tk, cap, scale_q in ((32, 8, 128, 4096, 4096, False), (20, 20, 64, 1000, 1500, True)):
        q, k, v = _case(heads, kv, hd, cap, 500 + tk)
        want = down(gpu.attn_decode_f16(q, k, v, heads, kv, hd, tk, cap, 0.09, scale_q, DecodeScratch()))
        out = torch.full((heads * hd,), float("nan"), device="cuda")
        got = down(gpu.attn_decode_f16_noalloc(q, k, v, heads, kv, hd, tk, cap, 0.09, scale_q, out))
        assert np.isfinite(got).all()
        assert np.array_equal(want.view(np.uint32), got.view(np.uint32)), (heads, kv, hd, tk)
        exact = oracle.decode_f64(oracle.seq(heads * hd, 500 + tk), oracle.through_f16(oracle.seq(kv * cap * hd,
                                  501 + tk)), oracle.through_f16(oracle.seq(kv * cap * hd, 502 + tk)), heads, kv, hd,
                                  tk, cap, 0.09, scale_q)
        assert np.abs(exact - got).max() / np.abs(exact).max() < 2e-5


def test_noalloc_decode_refuses_a_call_beyond_its_fixed_scratch(gpu):
    from ttsxabe_amd.gpu import ScratchLimit
    heads = kv = 300  # 300 kv heads' counters: more than the 256 the fixed scratch holds
    hd, tk, cap = 64, 64, 64
    q, k, v = _case(heads, kv, hd, cap, 900)
    out = torch.full((heads * hd,), 7.0, device="cuda")
    with pytest.raises(ScratchLimit):
        gpu.attn_decode_f16_noalloc(q, k, v, heads, kv, hd, tk, cap, 0.09, False, out)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()), "a refused call wrote its output"
