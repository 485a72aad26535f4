"""The multi-sequence step (sml_gpu_step_multi) on the GPU.

In the exact regime every sequence's logits equal decoding it alone, bit for
bit: the small-M GEMM gives each row the GEMV's arithmetic, and attention runs
per sequence over its own KV slot. The single-sequence reference runs with
the activation prologue fused but h quantized by its own launch (SML_FUSE=1),
which is the same arithmetic the batched step uses. In the default regime
for more than two sequences (per-256 activations) the step is checked
against the reference's own sml_forward_multi in its default regime.
"""
import numpy as np
import pytest

import sheep_amd as sa
from oracle import bind as ob

pytestmark = pytest.mark.gpu

PROMPTS = [[5, 17, 300], [1], [42, 42, 7, 1999, 3], [250, 11]]


def run_multi(path, n_vocab, steps):
    d = sa.Decoder(path, n_ctx=64)
    try:
        d.slots(len(PROMPTS))
        last = [d.prefill_slot(b, p, 0, n_vocab) for b, p in enumerate(PROMPTS)]
        toks = [int(np.argmax(l)) for l in last]
        pos = [len(p) for p in PROMPTS]
        out = []
        for _ in range(steps):
            lg = d.step_multi(toks, pos, list(range(len(PROMPTS))), n_vocab)
            out.append(lg)
            toks = [int(np.argmax(l)) for l in lg]
            pos = [p + 1 for p in pos]
        return last, out
    finally:
        d.close()


def run_alone(path, n_vocab, b, steps):
    d = sa.Decoder(path, n_ctx=64)
    try:
        last = d.prefill(np.array(PROMPTS[b], np.int32), 0, n_vocab)
        tok, pos, out = int(np.argmax(last)), len(PROMPTS[b]), []
        for _ in range(steps):
            lg = d.step(tok, pos, n_vocab)
            out.append(lg)
            tok, pos = int(np.argmax(lg)), pos + 1
        return last, out
    finally:
        d.close()


@pytest.mark.parametrize("kind", ["dense", "dense_perm", "moe", "hd64"])
def test_step_multi_equals_decoding_alone(tmp_path, kind, monkeypatch):
    """hd64: head_dim 64 (8 heads at hidden 512), whose batched step runs the
    4-wave attention of that head size."""
    monkeypatch.setenv("SML_FUSE", "1")
    monkeypatch.setenv("SML_MULTI", "exact")
    p = tmp_path / f"{kind}.ssf"
    extra = dict(n_expert=8, n_expert_used=2, moe_flags=1) if kind == "moe" else {}
    sa.synth_model(p, n_layer=2, n_embd=512, n_head=8 if kind == "hd64" else 4, n_head_kv=2, n_ff=1024,
                   n_vocab=2000, qkv_bias=True, random_perm=kind == "dense_perm", seed=70, **extra)
    steps = 6
    m_last, m_out = run_multi(p, 2000, steps)
    for b in range(len(PROMPTS)):
        a_last, a_out = run_alone(p, 2000, b, steps)
        np.testing.assert_array_equal(m_last[b], a_last, err_msg=f"prefill of slot {b}")
        for i in range(steps):
            np.testing.assert_array_equal(m_out[i][b], a_out[i], err_msg=f"sequence {b} step {i}")


@pytest.mark.parametrize("kind", ["dense", "moe"])
def test_step_multi_per32_regime_close_to_alone(tmp_path, kind, monkeypatch):
    """The per-32 regime without the exact flag (SML_MULTI_EXACT_MAX=16)
    agrees with decoding alone to float rounding: same greedy tokens, logits
    correlated to 0.9999."""
    monkeypatch.delenv("SML_MULTI", raising=False)
    monkeypatch.setenv("SML_MULTI_EXACT_MAX", "16")
    p = tmp_path / f"{kind}_mfma.ssf"
    extra = dict(n_expert=8, n_expert_used=2, moe_flags=1) if kind == "moe" else {}
    sa.synth_model(p, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000, seed=73, **extra)
    steps = 6
    m_last, m_out = run_multi(p, 2000, steps)
    for b in range(len(PROMPTS)):
        a_last, a_out = run_alone(p, 2000, b, steps)
        for i in range(steps):
            assert np.corrcoef(m_out[i][b], a_out[i])[0, 1] > 0.9999, (b, i)
            top = np.sort(a_out[i])[-2:]
            if top[1] - top[0] > 1e-2 * a_out[i].std():
                assert int(np.argmax(m_out[i][b])) == int(np.argmax(a_out[i])), (b, i)


def corr(a, b):
    return np.corrcoef(a, b)[0, 1]


@pytest.mark.skipif(not ob.have_ref(), reason="oracle/_ref (the reference's CPU engine) is not built")
@pytest.mark.parametrize("kind", ["dense", "dense_perm", "moe"])
def test_step_multi_per256_matches_reference(tmp_path, kind, monkeypatch):
    """The default regime for more than two sequences (per-256 activations,
    integer superblock sums) against the reference's sml_forward_multi in its
    default regime (rows-in-lanes on per-256 activations,
    sml/sml-run.c:2559-2599), each prompt read position by position on both
    sides, teacher-forced on the reference's tokens.

    Both sides compute the same integer sums but add floats in different
    orders, and a 1e-7 difference flips an int8 activation code now and then;
    one flipped code at the head's input moves the logits by ~1e-3 relative.
    So the regime is pinned by distance over the steps: the step's mean
    distance to the reference's per-256 logits is under a third of the
    reference's own per-32 stepping's distance to them (measured ~1/10 on
    this one-layer model). Per token: logits correlate to 0.9999 and the
    greedy token is the reference's outside the 1% tie rule."""
    monkeypatch.delenv("SML_MULTI", raising=False)
    monkeypatch.delenv("SML_MULTI_EXACT_MAX", raising=False)
    p = tmp_path / f"{kind}_sb.ssf"
    extra = dict(n_expert=8, n_expert_used=2, moe_flags=1) if kind == "moe" else {}
    sa.synth_model(p, n_layer=1, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000, qkv_bias=True,
                   random_perm=kind == "dense_perm", seed=74, **extra)
    ns, steps = len(PROMPTS), 8
    m = ob.RefMulti(p, 64, ns)
    alone = ob.RefMulti(p, 64, ns)          # the same sequences stepped one at a time, per 32
    d = sa.Decoder(p, n_ctx=64)
    d_gpu, d_regime = [], []
    try:
        d.slots(ns)
        toks, pos = [], []
        for b, prompt in enumerate(PROMPTS):
            for i, t in enumerate(prompt):
                lr = m.forward(b, t, i)
                alone.forward(b, t, i)
            lg = d.prefill_slot(b, prompt, 0, 2000)
            assert corr(lg, lr) > 0.9999, f"prefill of slot {b}"
            toks.append(int(np.argmax(lr)))
            pos.append(len(prompt))
        for i in range(steps):
            ref = m.step(toks, pos).astype(np.float64)
            got = d.step_multi(toks, pos, list(range(ns)), 2000).astype(np.float64)
            ex = np.stack([alone.forward(b, toks[b], pos[b]) for b in range(ns)]).astype(np.float64)
            d_gpu.append(np.sqrt(((got - ref) ** 2).mean() / (ref ** 2).mean()))
            d_regime.append(np.sqrt(((ex - ref) ** 2).mean() / (ref ** 2).mean()))
            for b in range(ns):
                g, r = got[b], ref[b]
                assert corr(g, r) > 0.9999, (b, i)
                top = np.sort(r)[-2:]
                if top[1] - top[0] > 1e-2 * r.std():
                    assert int(np.argmax(g)) == int(np.argmax(r)), (b, i)
            toks = [int(np.argmax(r)) for r in ref]
            pos = [q + 1 for q in pos]
    finally:
        d.close()
        m.close()
        alone.close()
    assert np.mean(d_gpu) < np.mean(d_regime) / 3, f"{np.mean(d_gpu):.3g} from per-256, per-32 is {np.mean(d_regime):.3g}"


def test_step_multi_greedy_tokens_match_oracle(tmp_path, monkeypatch):
    """The per-32 regime against the oracle's stepped decode."""
    monkeypatch.delenv("SML_MULTI", raising=False)
    monkeypatch.setenv("SML_MULTI_EXACT_MAX", "16")
    p = tmp_path / "multi_orc.ssf"
    sa.synth_model(p, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000, random_perm=True,
                   seed=71)
    steps = 10
    _, m_out = run_multi(p, 2000, steps)
    for b, prompt in enumerate(PROMPTS):
        om = ob.OracleModel(p, 64)
        try:
            for i, t in enumerate(prompt):
                lg = om.forward(t, i)
            pos, tok = len(prompt), int(np.argmax(lg))
            for i in range(steps):
                ref = om.forward(tok, pos)
                got = m_out[i][b]
                assert np.corrcoef(got, ref)[0, 1] > 0.999, (b, i)
                top = np.sort(ref)[-2:]
                if top[1] - top[0] > 1e-2 * ref.std():
                    assert int(np.argmax(got)) == int(np.argmax(ref)), (b, i)
                tok, pos = int(np.argmax(got)), pos + 1
        finally:
            om.close()


@pytest.mark.parametrize("ns", [2, 4])
def test_step_multi_graph_replays_equal_direct(tmp_path, ns, monkeypatch):
    """The batched step replays one captured HIP graph per (sequence count,
    regime). Six steps in a row, with host work and a synchronization
    between the replays, give every step's logits bit for bit as launching
    each kernel directly (SML_GRAPH=0)."""
    monkeypatch.delenv("SML_MULTI", raising=False)
    monkeypatch.delenv("SML_MULTI_EXACT_MAX", raising=False)
    p = tmp_path / "graph.ssf"
    sa.synth_model(p, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000, qkv_bias=True,
                   random_perm=True, seed=75, n_expert=8, n_expert_used=2, moe_flags=1)
    outs = {}
    for graph in ("0", "1"):
        monkeypatch.setenv("SML_GRAPH", graph)
        d = sa.Decoder(p, n_ctx=64)
        try:
            d.slots(ns)
            last = [d.prefill_slot(b, PROMPTS[b], 0, 2000) for b in range(ns)]
            toks = [int(np.argmax(l)) for l in last]
            pos = [len(PROMPTS[b]) for b in range(ns)]
            res = []
            for _ in range(6):
                lg = d.step_multi(toks, pos, list(range(ns)), 2000)
                res.append(lg)
                sa.sync()
                toks = [int(np.argmax(l)) for l in lg]
                pos = [q + 1 for q in pos]
            outs[graph] = res
        finally:
            d.close()
    for i in range(6):
        np.testing.assert_array_equal(outs["1"][i], outs["0"][i], err_msg=f"step {i}")


def test_step_multi_rejects_bad_arguments(tmp_path):
    p = tmp_path / "multi_bad.ssf"
    sa.synth_model(p, n_layer=1, n_embd=256, n_head=2, n_head_kv=1, n_ff=512, n_vocab=300, seed=72)
    d = sa.Decoder(p, n_ctx=16)
    try:
        assert sa.lib().sml_gpu_slots(17) == 0
        d.slots(2)
        out = np.zeros((2, 300), np.float32)
        I = sa.ctypes.c_int * 2
        f = sa.lib().sml_gpu_step_multi
        assert f(I(1, 2), I(0, 0), I(0, 0), 2, out.ctypes.data) == 0      # one slot twice
        assert f(I(1, 2), I(0, 16), I(0, 1), 2, out.ctypes.data) == 0     # position past n_ctx
        assert f(I(1, 300), I(0, 0), I(0, 1), 2, out.ctypes.data) == 0    # token past n_vocab
        assert f(I(1, 2), I(0, 0), I(0, 2), 2, out.ctypes.data) == 0      # slot not allocated
        assert f(I(1, 2), I(0, 0), I(0, 1), 2, out.ctypes.data) == 2
    finally:
        d.close()


@pytest.mark.parametrize("kind", ["dense", "moe"])
def test_step_multi_per256_merge_quantizes_as_its_own_launch(tmp_path, kind, monkeypatch):
    """In the per-256 regime the attention merge quantizes its output per 256
    values (two heads a superblock) for the o product; with
    SML_MERGE_Q256=0 the same quantization runs as its own launch over the
    merged output. Every step's logits are equal bit for bit."""
    monkeypatch.delenv("SML_MULTI", raising=False)
    monkeypatch.delenv("SML_MULTI_EXACT_MAX", raising=False)
    p = tmp_path / f"merge_{kind}.ssf"
    extra = dict(n_expert=8, n_expert_used=2, moe_flags=1) if kind == "moe" else {}
    sa.synth_model(p, n_layer=2, n_embd=1024, n_head=8, n_head_kv=2, n_ff=2048, n_vocab=2000, qkv_bias=True,
                   seed=76, **extra)
    outs = {}
    for fused in ("0", "1"):
        monkeypatch.setenv("SML_MERGE_Q256", fused)
        print(f"per-256 merge {kind} fused {fused}", flush=True)
        _, outs[fused] = run_multi(p, 2000, 6)
    for i in range(6):
        np.testing.assert_array_equal(outs["1"][i], outs["0"][i], err_msg=f"step {i}")


@pytest.mark.parametrize("heads", [(8, 2), (12, 2), (8, 8), (16, 2)])
def test_step_multi_spread_attention_equals_one_entry_body(tmp_path, heads, monkeypatch):
    """The batched decode attention with its q, k, v and RoPE inputs spread
    over the workgroup (sml_attnb) against the one-entry body's 4-wave form
    (SML_ATTNB=0): six sequences whose positions cross split boundaries
    (1..384 of a 512-position cache), 1, 4, 6 and 8 query heads per kv head;
    every step's logits are equal bit for bit."""
    monkeypatch.delenv("SML_MULTI", raising=False)
    monkeypatch.delenv("SML_MULTI_EXACT_MAX", raising=False)
    nh, nkv = heads
    p = tmp_path / f"spread_{nh}_{nkv}.ssf"
    sa.synth_model(p, n_layer=2, n_embd=nh * 128, n_head=nh, n_head_kv=nkv, n_ff=1024, n_vocab=2000,
                   qkv_bias=True, seed=77)
    lens = [1, 127, 128, 129, 300, 383]
    rng = np.random.default_rng(77)
    prompts = [rng.integers(0, 2000, n).astype(np.int32) for n in lens]
    outs = {}
    for spread in ("0", "1"):
        monkeypatch.setenv("SML_ATTNB", spread)
        print(f"spread attention {heads} {spread}", flush=True)
        d = sa.Decoder(p, n_ctx=512)
        try:
            d.slots(len(lens))
            last = [d.prefill_slot(b, pr, 0, 2000) for b, pr in enumerate(prompts)]
            toks, pos, out = [int(np.argmax(l)) for l in last], list(lens), []
            for _ in range(3):
                lg = d.step_multi(toks, pos, list(range(len(lens))), 2000)
                out.append(lg)
                toks = [int(np.argmax(l)) for l in lg]
                pos = [x + 1 for x in pos]
            outs[spread] = out
        finally:
            d.close()
    for i in range(3):
        np.testing.assert_array_equal(outs["1"][i], outs["0"][i], err_msg=f"step {i}")


def test_step_multi_split_k_down_product(tmp_path, monkeypatch):
    """The per-256 batched step of 12 sequences (the matrix-core products
    take more than 8) with a 5120-wide FFN: the down product (20
    superblocks) runs split in 4 slices, its residual added by
    sml_gemm_ksum. Against the one-pass kernel (SML_MGEMM_KS=1) every step's
    logits correlate to 0.99999 and keep their top-1 wherever the top two
    are more than 1% of a logit s.d. apart."""
    monkeypatch.delenv("SML_MULTI", raising=False)
    monkeypatch.delenv("SML_MULTI_EXACT_MAX", raising=False)
    p = tmp_path / "splitk.ssf"
    sa.synth_model(p, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=5120, n_vocab=2000, qkv_bias=True,
                   seed=78)
    prompts = [[(7 * b + 3 * j + 1) % 2000 for j in range(1 + b % 5)] for b in range(12)]
    outs, forced = {}, None
    for ks in ("1", "4"):
        monkeypatch.setenv("SML_MGEMM_KS", ks)
        print(f"split-k {ks}", flush=True)
        d = sa.Decoder(p, n_ctx=64)
        try:
            d.slots(len(prompts))
            last = [d.prefill_slot(b, pr, 0, 2000) for b, pr in enumerate(prompts)]
            toks, pos, out, used = [int(np.argmax(l)) for l in last], [len(pr) for pr in prompts], [], []
            for i in range(4):
                if forced is not None:
                    toks = forced[i]                # teacher-forced on the one-pass run's ids
                used.append(list(toks))
                lg = d.step_multi(toks, pos, list(range(len(prompts))), 2000)
                out.append(lg)
                toks = [int(np.argmax(l)) for l in lg]
                pos = [x + 1 for x in pos]
            outs[ks], forced = out, used
        finally:
            d.close()
    differ = False
    for i in range(4):
        for b in range(len(prompts)):
            a, r = outs["4"][i][b], outs["1"][i][b]
            differ |= not np.array_equal(a, r)
            assert corr(a, r) > 0.99999, (i, b)
            top = np.sort(r)[-2:]
            if top[1] - top[0] > 1e-2 * r.std():
                assert int(np.argmax(a)) == int(np.argmax(r)), (i, b)
    assert differ, "the split form did not run"


def test_step_multi_split_k_sums_fused_with_the_next_norm(tmp_path, monkeypatch):
    """The per-256 batched step leaves the split-K down product's slice sums
    to the next layer's (and the head's) norm, which adds them as it
    normalizes and quantizes each row (sml_ksum_normq). Every step's logits
    equal the two launches' (SML_KSUM_NORMQ=0: sml_gemm_ksum, then
    sml_normq2) bit for bit: 12 sequences, a 1536-wide residual (rows that
    are no multiple of 1024 values), permuted columns and q/k/v biases. The
    one-pass product (SML_MGEMM_KS=1) differs, so the split form ran."""
    monkeypatch.delenv("SML_MULTI", raising=False)
    monkeypatch.delenv("SML_MULTI_EXACT_MAX", raising=False)
    p = tmp_path / "ksumq.ssf"
    sa.synth_model(p, n_layer=3, n_embd=1536, n_head=12, n_head_kv=4, n_ff=5120, n_vocab=2000, qkv_bias=True,
                   random_perm=True, seed=79)
    prompts = [[(5 * b + 3 * j + 2) % 2000 for j in range(1 + b % 4)] for b in range(12)]
    outs = {}
    for name, fused, ks in (("two", "0", "4"), ("fused", "1", "4"), ("one-pass", "1", "1")):
        monkeypatch.setenv("SML_KSUM_NORMQ", fused)
        monkeypatch.setenv("SML_MGEMM_KS", ks)
        print(name, flush=True)
        d = sa.Decoder(p, n_ctx=64)
        try:
            d.slots(len(prompts))
            last = [d.prefill_slot(b, pr, 0, 2000) for b, pr in enumerate(prompts)]
            toks, pos, out = [int(np.argmax(l)) for l in last], [len(pr) for pr in prompts], []
            for i in range(3):
                lg = d.step_multi(toks, pos, list(range(len(prompts))), 2000)
                out.append(lg)
                toks = [int(np.argmax(l)) for l in lg]
                pos = [x + 1 for x in pos]
            outs[name] = out
        finally:
            d.close()
    for i in range(3):
        a, r = outs["fused"][i], outs["two"][i]
        bad = np.flatnonzero(a.view(np.uint32) != r.view(np.uint32))
        assert bad.size == 0, (i, bad.size, bad[:4])
    assert not np.array_equal(outs["fused"][0], outs["one-pass"][0]), "the split form did not run"
