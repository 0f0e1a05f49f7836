"""The XCD-local split hand-off checks itself.

The decode's in-launch merge keeps a head's splits on one XCD when the plan
allows (partials in that XCD's L2, no coherent stores). That relies on the
dispatcher putting workgroups L and L + 8k on one XCD; every workgroup adds
its XCC id (and its square) to the head's arrival counter, so the merging
workgroup knows whether the head really stayed on one XCD. Here: the mode on
and off give the same bits, and XCC ids faked from the host to differ within
a head turn every merged head into NaN, never into a silently wrong context,
and leave the counters clean.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.util import down, up, up_f16

pytestmark = pytest.mark.gpu


def _c2(gpu, tiled, s=None):
    from ttsxabe_amd.gpu import DecodeScratch, TiledCache16
    heads, kv, hd, tk, cap = 32, 8, 128, 4096, 4096
    q = up(oracle.seq(heads * hd, 41))
    k = up_f16(oracle.seq(kv * cap * hd, 42))
    v = up_f16(oracle.seq(kv * cap * hd, 43))
    s = s or DecodeScratch()
    if tiled:
        t = TiledCache16(kv, hd, cap)
        gpu.t16_from_ref(k, v, t, tk)
        return lambda: down(gpu.attn_decode_t16(q, t, heads, tk, 0.088, False, s))
    return lambda: down(gpu.attn_decode_f16(q, k, v, heads, kv, hd, tk, cap, 0.088, False, s))


@pytest.mark.parametrize("tiled", [False, True])
def test_the_xcd_local_hand_off_matches_the_coherent_one(gpu, tiled, monkeypatch):
    run = _c2(gpu, tiled)
    local = run()
    monkeypatch.setenv("LLMTIE_DECODE_XCD", "0")
    coherent = run()
    assert np.isfinite(local).all()
    assert np.array_equal(local.view(np.uint32), coherent.view(np.uint32))


def test_a_head_spread_over_xcds_is_nan_and_reported(gpu):
    """Faked XCC ids (the test hook) make every merged head fail the check:
    its context is NaN, the scratch's status says so (and is cleared by
    reading it), the next call through the scratch is refused with the same
    status before it launches, and the counters are left clean."""
    from ttsxabe_amd import _lib
    from ttsxabe_amd.gpu import DecodeScratch, SplitHeadLost
    s = DecodeScratch()
    run = _c2(gpu, True, s)
    good = run()
    s.check()
    _lib.lib().llmtie_debug_fake_xcc(1)  # workgroup L reports XCC id (L / 8) % 8
    try:
        bad = run()
    finally:
        _lib.lib().llmtie_debug_fake_xcc(0)
    assert np.isnan(bad).all(), "every head of C2 is merged across splits"
    with pytest.raises(SplitHeadLost):
        run()  # refused: the earlier call lost heads
    again = run()  # the refusal cleared the status; the counters were reset by the NaN path
    assert np.array_equal(good.view(np.uint32), again.view(np.uint32))
    _lib.lib().llmtie_debug_fake_xcc(1)
    try:
        run()
    finally:
        _lib.lib().llmtie_debug_fake_xcc(0)
    torch.cuda.synchronize()
    with pytest.raises(SplitHeadLost):
        s.check()
    s.check()  # cleared
