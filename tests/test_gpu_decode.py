"""The sml-gpu.h forward pass on the GPU against the oracle's decoder.

Logits agree to the size an int8 activation-code flip makes (the quantized
activations turn last-bit float differences into one-code steps; see the
reference's own per-position correlation grading, sml/sml-gpu-fwd.c:2565-2601).
Greedy token ids must be identical; a mismatch reports the oracle's top-2
margin against the reference's 1%-of-s.d. tie rule as the diagnostic.
"""
import numpy as np
import pytest

import sheep_amd as sa
from oracle import bind as ob

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    p = tmp_path_factory.mktemp("dec") / "tiny.ssf"
    sa.synth_model(p, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000,
                   qkv_bias=True, random_perm=True, seed=31)
    return p


@pytest.fixture(scope="module")
def tiny_inorder(tmp_path_factory):
    """No permutations: the q/k/v and gate/up GEMVs compute their activations
    in their prologues, attention quantizes o's input and SwiGLU quantizes h."""
    p = tmp_path_factory.mktemp("dec") / "tiny_inorder.ssf"
    sa.synth_model(p, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000,
                   qkv_bias=True, random_perm=False, seed=32)
    return p


@pytest.fixture(scope="module")
def qwenish(tmp_path_factory):
    """Qwen2.5-1.5B layer shapes (hidden 1536, FFN 8960, 12/2 heads, q/k/v bias,
    tied head) with 4 layers and a 32000 vocabulary."""
    p = tmp_path_factory.mktemp("dec") / "qwenish.ssf"
    sa.synth_model(p, n_layer=4, n_embd=1536, n_head=12, n_head_kv=2, n_ff=8960, n_vocab=32000,
                   rope_theta=1e6, qkv_bias=True, tied=True, random_perm=True, seed=1002)
    return p


def greedy_oracle(path, tok, n, n_ctx):
    m = ob.OracleModel(path, n_ctx)
    toks, logits = [tok], []
    for pos in range(n):
        lg = m.forward(toks[-1], pos)
        logits.append(lg)
        toks.append(int(np.argmax(lg)))
    m.close()
    return toks, logits


def tie_margin(lg):
    top = np.sort(lg)[-2:]
    return (top[1] - top[0]) / lg.std()


def check_tokens(gpu_toks, orc_toks, orc_logits):
    for i, (a, b) in enumerate(zip(gpu_toks, orc_toks)):
        if a != b:
            m = tie_margin(orc_logits[i])
            pytest.fail(f"step {i}: gpu {a} oracle {b}; oracle top-2 margin {m:.4f} s.d. "
                        f"({'inside' if m <= 0.01 else 'outside'} the reference's 1% tie rule)")


@pytest.mark.parametrize("graph", ["1", "0"])
def test_teacher_forced_logits(tiny, graph, monkeypatch):
    monkeypatch.setenv("SML_GRAPH", graph)
    toks, logits = greedy_oracle(tiny, 3, 12, 64)
    d = sa.Decoder(tiny, n_ctx=64)
    try:
        for pos in range(12):
            lg = d.step(toks[pos], pos, 2000)
            ref = logits[pos]
            assert np.corrcoef(lg, ref)[0, 1] > 0.999, pos
            assert np.abs(lg - ref).max() <= 3e-2 * np.abs(ref).max(), pos
    finally:
        d.close()


def test_greedy_tokens_tiny(tiny):
    n = 40
    toks, logits = greedy_oracle(tiny, 11, n, 64)
    d = sa.Decoder(tiny, n_ctx=64)
    try:
        out = d.generate(11, 0, n)
    finally:
        d.close()
    check_tokens(list(out), toks[1:], logits)


def test_greedy_tokens_inorder(tiny_inorder):
    n = 40
    toks, logits = greedy_oracle(tiny_inorder, 7, n, 64)
    d = sa.Decoder(tiny_inorder, n_ctx=64)
    try:
        out = d.generate(7, 0, n)
    finally:
        d.close()
    check_tokens(list(out), toks[1:], logits)


@pytest.mark.parametrize("model", ["tiny", "tiny_inorder"])
def test_fusions_do_not_change_logits(model, request, monkeypatch):
    """With the fused prologues and h quantization switched off, each layer
    runs the separate normq launches instead. The prologue's activations are
    the same bits; the h-quantizing SwiGLU sums each row over 16 lanes instead
    of 64, which moves h by float rounding (and can move an int8 code of h by
    one step). The logits agree closely and pick the same token."""
    path = request.getfixturevalue(model)
    outs = []
    for fuse in ("3", "0"):
        monkeypatch.setenv("SML_FUSE", fuse)
        d = sa.Decoder(path, n_ctx=64)
        try:
            outs.append([d.step(t, i, 2000).copy() for i, t in enumerate([3, 17, 250, 9, 1999])])
        finally:
            d.close()
    for a, b in zip(*outs):
        assert np.corrcoef(a, b)[0, 1] > 0.9999
        assert int(np.argmax(a)) == int(np.argmax(b))


def test_generate_equals_stepping_and_prefill(tiny):
    d = sa.Decoder(tiny, n_ctx=64)
    try:
        gen = d.generate(5, 0, 16)
        # stepping the same positions with the generated tokens reproduces them
        seq = [5] + list(gen)
        stepped = [int(np.argmax(d.step(seq[i], i, 2000))) for i in range(16)]
        assert stepped == list(gen)
        # a prompt read at once continues exactly as stepping did
        lg = d.prefill(np.array(seq[:10], np.int32), 0, 2000)
        assert int(np.argmax(lg)) == gen[9]
    finally:
        d.close()


@pytest.fixture(scope="module")
def moe_model(tmp_path_factory):
    p = tmp_path_factory.mktemp("dec") / "moe_pf.ssf"
    sa.synth_model(p, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000, n_expert=8,
                   n_expert_used=2, moe_flags=1, random_perm=True, seed=62)
    return p


@pytest.mark.parametrize("model", ["tiny", "tiny_inorder", "qwenish", "moe_model"])
def test_batched_prompt_equals_stepping(model, request):
    """Batched prompt reading (level 1, the default): chunks of 16 positions
    through the small-M GEMM and the causal attention read a prompt exactly
    as stepping it does -- the logits of the last id bit for bit, for a first
    part and for a continuation of that prefix (37 ids: ragged chunks), and
    the same greedy continuation. Level 2 (Q4 on MFMA) agrees to float
    rounding."""
    p = request.getfixturevalue(model)
    V = 32000 if model == "qwenish" else 2000
    ids = np.random.default_rng(17).integers(0, V, 37).astype(np.int32)
    outs = {}
    for level in (0, 1, 2):
        d = sa.Decoder(p, n_ctx=96)
        try:
            d.prompt_mode(level)
            a = d.prefill(ids[:20], 0, V)
            b = d.prefill(ids[20:], 20, V)
            gen = list(d.generate(int(np.argmax(b)), 37, 8))
            outs[level] = (a, b, gen)
        finally:
            d.close()
    for i in range(2):
        np.testing.assert_array_equal(outs[1][i], outs[0][i], err_msg=f"level 1, part {i}")
    assert outs[1][2] == outs[0][2]
    for i in range(2):
        ref = outs[0][i]
        assert np.corrcoef(outs[2][i], ref)[0, 1] > 0.9999, f"level 2, part {i}"
        if tie_margin(ref) > 0.01:
            assert int(np.argmax(outs[2][i])) == int(np.argmax(ref)), f"level 2, part {i}"


@pytest.mark.parametrize("n", [16, 17, 33, 64])
def test_batched_prompt_fills_context(tiny, n):
    """Prompts that end exactly at n_ctx (the last position's K/V row is the
    cache's last), with whole and ragged chunks: level 1 equals stepping bit
    for bit, level 2 within float rounding; a prompt past n_ctx is refused."""
    ids = np.random.default_rng(n).integers(0, 2000, n).astype(np.int32)
    outs = {}
    for level in (0, 1, 2):
        d = sa.Decoder(tiny, n_ctx=n)
        try:
            d.prompt_mode(level)
            outs[level] = d.prefill(ids, 0, 2000)
            assert not sa.lib().sml_gpu_prefill(ids.ctypes.data_as(sa.P(sa.c_int)), 1, n)
        finally:
            d.close()
    np.testing.assert_array_equal(outs[1], outs[0])
    assert np.corrcoef(outs[2], outs[0])[0, 1] > 0.9999


def test_batched_prompt_into_other_slots(tiny):
    """sml_gpu_prefill_slot batched into slots 1 and 2 (levels 1 and 2) leaves
    each slot's cache as reading the prompt a token at a time does: the
    following multi-sequence step equals the one after stepped prompts, bit
    for bit."""
    prompts = [np.random.default_rng(s).integers(0, 2000, 21 + s).astype(np.int32) for s in range(3)]
    res = {}
    for level in (0, 1, 2):
        d = sa.Decoder(tiny, n_ctx=64)
        try:
            d.prompt_mode(level)
            d.slots(3)
            last = [d.prefill_slot(b, p, 0, 2000) for b, p in enumerate(prompts)]
            toks = [int(np.argmax(l)) for l in last]
            pos = [len(p) for p in prompts]
            steps = [d.step_multi(toks, pos, [0, 1, 2], 2000)]
            res[level] = (last, steps)
        finally:
            d.close()
    for b in range(3):
        np.testing.assert_array_equal(res[1][0][b], res[0][0][b], err_msg=f"slot {b} prompt logits")
        np.testing.assert_array_equal(res[1][1][0][b], res[0][1][0][b], err_msg=f"slot {b} step")
        assert np.corrcoef(res[2][0][b], res[0][0][b])[0, 1] > 0.9999


def test_greedy_tokens_qwen_layers(qwenish):
    n = 24
    toks, logits = greedy_oracle(qwenish, 100, n, 128)
    d = sa.Decoder(qwenish, n_ctx=128)
    try:
        out = d.generate(100, 0, n)
    finally:
        d.close()
    check_tokens(list(out), toks[1:], logits)


@pytest.mark.parametrize("perm", [False, True])
def test_greedy_tokens_moe(tmp_path, perm):
    """A Mixtral-shaped decoder (8 experts, top-2, softmax over the chosen):
    routed experts on the GPU, tokens identical to the oracle."""
    p = tmp_path / "moe.ssf"
    sa.synth_model(p, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000, n_expert=8,
                   n_expert_used=2, moe_flags=1, random_perm=perm, seed=60 + int(perm))
    n = 24
    toks, logits = greedy_oracle(p, 9, n, 64)
    d = sa.Decoder(p, n_ctx=64)
    try:
        for pos in range(4):
            lg = d.step(toks[pos], pos, 2000)
            assert np.corrcoef(lg, logits[pos])[0, 1] > 0.999, pos
        out = d.generate(9, 0, n)
    finally:
        d.close()
    check_tokens(list(out), toks[1:], logits)


def test_bounds_and_reopen(tiny):
    d = sa.Decoder(tiny, n_ctx=32)
    try:
        assert not sa.lib().sml_gpu_step(1, 32)
        assert not sa.lib().sml_gpu_step(2000, 0)
        assert sa.lib().sml_gpu_generate(1, 30, 5, (sa.ctypes.c_int * 5)()) == -1
    finally:
        d.close()
    d = sa.Decoder(tiny, n_ctx=32)
    d.close()
