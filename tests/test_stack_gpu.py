"""The attention path inside a random-init Llama stack: greedy decode on the
GPU (ttsxabe_amd.stack: torch projections, this library's RoPE, cache writes,
growth and attention) against the CPU restatement of the same stack
(oracle/stack.py), token by token.

The reference's own end-to-end check is the chat model's argmax against a
captured run of the original (crates/llmtie-chat/tests/stepwise.rs); with no
checkpoint here, the same check runs on random weights. The prompt is 250
tokens so decoding crosses the 256-position cache capacity and exercises the
growth path. The GPU rounds q and the probabilities to f16 in the prefill
(the reference's flash arithmetic), so logits agree to ~1e-3 of their scale,
not bit for bit. The argmax must be identical at every step (the north
star's rule); steps whose CPU top-two margin is inside twice the measured
logit error are counted and printed as near-ties, but they too must agree.
Both sides continue from the CPU's token.
"""
import numpy as np
import pytest

from oracle.stack import CpuStack, StackConfig, random_weights

from tests.configs import SEED

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("layout", ["reference", "tiled"])
def test_random_llama_stack_decodes_like_the_cpu(gpu, layout):
    from ttsxabe_amd.stack import LlamaStack
    cfg = StackConfig()
    w = random_weights(cfg, SEED)
    cpu = CpuStack(cfg, w)
    dev = LlamaStack(gpu, cfg, w, layout)
    rng = np.random.default_rng(SEED + 1)
    ids = [int(t) for t in rng.integers(0, cfg.vocab, 250)]
    ties = 0
    for step in range(12):
        lc = cpu.forward(ids)
        lg = dev.forward(ids).float().cpu().numpy()
        scale = float(np.abs(lc).max())
        err = float(np.abs(lc - lg).max())
        assert err < 5e-3 * scale, f"{layout} step {step}: logit error {err:.3g} of scale {scale:.3g}"
        top_c, top_g = int(lc.argmax()), int(lg.argmax())
        srt = np.sort(lc)
        margin = float(srt[-1] - srt[-2])
        if margin <= 2 * err + 1e-6:
            ties += 1
        assert top_g == top_c, f"{layout} step {step}: GPU argmax {top_g} != CPU {top_c} (margin {margin:.3g})"
        ids = [top_c]
    print(f"{layout}: {ties} of 12 steps had a top-two margin inside twice the logit error", flush=True)
    assert dev.past == cpu.past == 261 and dev.cap == 512


@pytest.mark.parametrize("layout", ["reference", "tiled"])
def test_a_gguf_llama_decodes_like_the_cpu(gpu, layout, tmp_path):
    """The same check on weights read back from a llama.cpp-style GGUF (F16
    and Q8_0 matrices, q/k rows permuted for interleaved RoPE, a Llama-3
    rope_freqs table): the binding must undo the permutation and carry the
    frequency divisors to this library's RoPE for the argmax to hold."""
    from ttsxabe_amd.llama_gguf import load_llama_gguf
    from ttsxabe_amd.stack import LlamaStack
    from tests.test_gguf import llama_gguf
    cfg = StackConfig()
    w = random_weights(cfg, SEED + 7)
    held = llama_gguf(tmp_path / "m.gguf", cfg, w, rope_freqs=np.linspace(1.0, 8.0, cfg.head_dim // 2,
                                                                           dtype=np.float32))
    c, wl = load_llama_gguf(tmp_path / "m.gguf")
    cpu = CpuStack(c, held)
    dev = LlamaStack(gpu, c, wl, layout)
    rng = np.random.default_rng(SEED + 8)
    ids = [int(t) for t in rng.integers(0, c.vocab, 40)]
    for step in range(6):
        lc = cpu.forward(ids)
        lg = dev.forward(ids).float().cpu().numpy()
        scale = float(np.abs(lc).max())
        err = float(np.abs(lc - lg).max())
        assert err < 5e-3 * scale, f"{layout} step {step}: logit error {err:.3g} of scale {scale:.3g}"
        assert int(lg.argmax()) == int(lc.argmax()), f"{layout} step {step}"
        ids = [int(lc.argmax())]
