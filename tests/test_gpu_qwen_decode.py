"""Full-size decoders on the GPU against the reference's own CPU engine.

Qwen2.5-1.5B-shaped decoder on the GPU against the reference's own
CPU engine (oracle/_ref: sml/sml-run.c sml_forward built from the
reference's sources): 28 layers, hidden 1536, FFN 8960, 12 query / 2 KV
heads, head_dim 128, RoPE theta 1e6, q/k/v bias, tied 151936-token head,
random column permutations, random-init Q4 weights. A 2048-id random prompt
is read position by position on both sides, then 64 greedy tokens follow;
the token ids must be identical at every step.

The reference reads the prompt with sml_forward, one position at a time, as
the GPU does (its batched sml_prefill quantizes activations per 256 and
would start the continuation from a different state).
"""
import os

import numpy as np
import pytest

import sheep_amd as sa
from oracle import bind as ob

pytestmark = pytest.mark.gpu

PROMPT, STEPS = 2048, 64
QWEN = dict(n_layer=28, n_embd=1536, n_head=12, n_head_kv=2, n_ff=8960, n_vocab=151936, rope_theta=1e6,
            rms_eps=1e-6, qkv_bias=True, tied=True, random_perm=True, nbits=4, seed=2025)


def tie_margin(lg):
    top = np.sort(lg)[-2:]
    return (top[1] - top[0]) / lg.std()


@pytest.mark.timeout(600)
@pytest.mark.skipif(not ob.have_ref(), reason="oracle/_ref (the reference's CPU engine) is not built")
def test_qwen25_1p5b_prompt2048_greedy64(tmp_path):
    p = tmp_path / "qwen25_1p5b.ssf"
    sa.synth_model(p, n_ctx_train=4096, **QWEN)
    V = QWEN["n_vocab"]
    prompt = np.random.default_rng(7).integers(0, V, PROMPT).astype(np.int32)
    n_ctx = PROMPT + STEPS

    d = sa.Decoder(p, n_ctx=n_ctx)
    try:
        lg = d.prefill(prompt, 0, V)
        first = int(np.argmax(lg))
        gpu = [first] + [int(t) for t in d.generate(first, PROMPT, STEPS - 1)]
    finally:
        d.close()

    m = ob.RefModel(p, n_ctx, threads=min(16, os.cpu_count() or 1))
    try:
        for pos, tok in enumerate(prompt):
            lg = m.forward(int(tok), pos)
        ref, logits = [], []
        for pos in range(PROMPT, PROMPT + STEPS):
            logits.append(lg)
            ref.append(int(np.argmax(lg)))
            if pos + 1 < PROMPT + STEPS:
                lg = m.forward(ref[-1], pos)
    finally:
        m.close()

    for i, (a, b) in enumerate(zip(gpu, ref)):
        if a != b:
            mg = tie_margin(logits[i])
            pytest.fail(f"step {i}: gpu {a} reference {b}; reference top-2 margin {mg:.4f} s.d. "
                        f"({'inside' if mg <= 0.01 else 'outside'} the reference's 1% tie rule)")
    assert len(gpu) == STEPS


LLAMA = dict(n_layer=32, n_embd=4096, n_head=32, n_head_kv=8, n_ff=14336, n_vocab=128256, rope_theta=500000.0,
             rms_eps=1e-5, qkv_bias=False, tied=False, random_perm=False, nbits=4, seed=1003)


@pytest.mark.timeout(600)
@pytest.mark.skipif(not ob.have_ref(), reason="oracle/_ref (the reference's CPU engine) is not built")
def test_llama3_8b_prompt1024_greedy64(tmp_path):
    """The Llama-3-8B-shaped decoder of the throughput workload (32 layers,
    hidden 4096, FFN 14336, 32/8 heads, untied 128256-token head, no
    permutations): a 1024-id prompt, then 64 greedy tokens identical to the
    reference's engine."""
    p = tmp_path / "llama3_8b.ssf"
    sa.synth_model(p, n_ctx_train=4096, **LLAMA)
    V, prompt_n = LLAMA["n_vocab"], 1024
    prompt = np.random.default_rng(11).integers(0, V, prompt_n).astype(np.int32)
    n_ctx = prompt_n + STEPS
    d = sa.Decoder(p, n_ctx=n_ctx)
    try:
        first = int(np.argmax(d.prefill(prompt, 0, V)))
        gpu = [first] + [int(t) for t in d.generate(first, prompt_n, STEPS - 1)]
    finally:
        d.close()
    m = ob.RefModel(p, n_ctx, threads=min(16, os.cpu_count() or 1))
    try:
        for pos, tok in enumerate(prompt):
            lg = m.forward(int(tok), pos)
        ref, logits = [], []
        for pos in range(prompt_n, prompt_n + STEPS):
            logits.append(lg)
            ref.append(int(np.argmax(lg)))
            if pos + 1 < prompt_n + STEPS:
                lg = m.forward(ref[-1], pos)
    finally:
        m.close()
    for i, (a, b) in enumerate(zip(gpu, ref)):
        if a != b:
            mg = tie_margin(logits[i])
            pytest.fail(f"step {i}: gpu {a} reference {b}; reference top-2 margin {mg:.4f} s.d. "
                        f"({'inside' if mg <= 0.01 else 'outside'} the reference's 1% tie rule)")
