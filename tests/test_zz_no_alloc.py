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


_FIRST_CALL_IN_CAPTURE = r"""
import sys
sys.path.insert(0, sys.argv[1])
import numpy as np, torch
import oracle
from ttsxabe_amd.gpu import DecodeScratch, Gpu
g = Gpu(0)
heads, kv, hd, tk, cap = 32, 8, 128, 4096, 4096
q = torch.from_numpy(oracle.seq(heads * hd, 71)).cuda()
k = torch.from_numpy(oracle.f32_to_f16(oracle.seq(kv * cap * hd, 72)).view(np.float16)).cuda()
v = torch.from_numpy(oracle.f32_to_f16(oracle.seq(kv * cap * hd, 73)).view(np.float16)).cuda()
want = g.attn_decode_f16(q, k, v, heads, kv, hd, tk, cap, 0.09, False, DecodeScratch()).cpu()
out = torch.full((heads * hd,), float("nan"), device="cuda")
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(s):
    with torch.cuda.graph(graph, stream=s):  # the process's first no-allocation call
        g.attn_decode_f16_noalloc(q, k, v, heads, kv, hd, tk, cap, 0.09, False, out)
torch.cuda.current_stream().wait_stream(s)
for rep in range(4):
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    got = out.cpu()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32)), f"replay {rep}"
    (q * 2).sum().item()  # eager work between replays
print("ok")
"""


def test_noalloc_first_call_under_capture_in_a_fresh_process(gpu):
    """The fixed scratch needs no clearing launch (it is zero at load), so a
    process whose first no-allocation call is made under stream capture
    records only the decode; every replay matches the scratch-taking decode."""
    import subprocess
    import sys
    from pathlib import Path
    root = str(Path(__file__).resolve().parent.parent)
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE, root], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout[-2000:] + r.stderr[-2000:]
