"""Pinning the CPU oracle (oracle/sml_oracle.c).

Each restated function is checked three ways where they apply: against the
golden vectors the reference build wrote (tests/golden/), against the
reference's own CPU path when it is built here (oracle/_ref), and against what
the mathematics fixes (closed forms, brute force in float64, invariants) --
chosen so that a dropped term, a wrong index or a swapped plane fails.
"""
import ctypes
import hashlib
import os

import numpy as np
import pytest

import sheep_amd as sa
from oracle import bind as ob
from sheep_amd.ssf import SSF

GOLD = os.path.join(os.path.dirname(__file__), "golden")
needs_ref = pytest.mark.skipif(not ob.have_ref(), reason="reference CPU build not present")


def f16(u16):
    return np.asarray(u16, np.uint16).view(np.float16).astype(np.float32)


# ------------------------------------------------------------ activations

def test_quantize_act_golden():
    g = np.load(os.path.join(GOLD, "act_quant.npz"))
    for i in range(2):
        for per256 in (0, 1):
            q, s, u = ob.quantize_act(g[f"x{i}"], per256=bool(per256))
            np.testing.assert_array_equal(q, g[f"q{i}_{per256}"])
            np.testing.assert_array_equal(s, g[f"s{i}_{per256}"])
            np.testing.assert_array_equal(u, g[f"u{i}_{per256}"])


@needs_ref
@pytest.mark.parametrize("seed", range(6))
def test_quantize_act_matches_reference(seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal(4096) * 10.0 ** rng.uniform(-3, 3)).astype(np.float32)
    x[rng.integers(0, 4096, 50)] = np.round(x[rng.integers(0, 4096, 50)])  # integers hit exact halves often
    for per256 in (False, True):
        for a, b in zip(ob.quantize_act(x, per256), ob.ref_quantize_act(x, per256)):
            np.testing.assert_array_equal(a, b)


def test_quantize_act_closed_form():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(2048).astype(np.float32)
    q, s, u = ob.quantize_act(x)
    g = x.reshape(-1, 32)
    amax = np.abs(g).max(1)
    np.testing.assert_array_equal(s, (amax / np.float32(127)).astype(np.float32))
    inv = (np.float32(1) / s).astype(np.float32)
    want = np.clip(np.rint((g * inv[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    np.testing.assert_array_equal(q.reshape(-1, 32), want)
    np.testing.assert_array_equal(u, want.astype(np.int32).sum(1))
    # the group maximum always lands on +-127
    assert (np.abs(q.reshape(-1, 32)).max(1) == 127).all()


# ------------------------------------------------------------ codes and GEMV per width

@pytest.mark.parametrize("nb", range(2, 9))
def test_widths_golden(tmpdir_s, nb):
    g = np.load(os.path.join(GOLD, "widths.npz"))
    p = tmpdir_s / f"gold{nb}.ssf"
    sa.synth_matrix(p, 16, 256, nbits=nb, random_perm=True, seed=100 + nb)
    assert hashlib.sha256(p.read_bytes()).digest() == g[f"sha{nb}"].tobytes(), "synthetic file drifted"
    t = SSF(p)["w"]
    deq = np.stack([ob.dequant_row(t, r) for r in range(16)])
    np.testing.assert_array_equal(deq, g[f"deq{nb}"])
    q, s, u = ob.quantize_act(g[f"x{nb}"])
    y = ob.matvec(t, q, s, u)
    ref = g[f"y{nb}"]
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("nb", range(2, 9))
def test_codes_closed_form(tmpdir_s, nb):
    """dequant == code*step + min with step/min from the fields; brute-force
    GEMV in float64 over the dequantized row agrees with the oracle GEMV."""
    p = tmpdir_s / f"cf{nb}.ssf"
    sa.synth_matrix(p, 12, 384, nbits=nb, random_perm=True, seed=40 + nb)
    t = SSF(p)["w"]
    ng = 384 // 32
    sd = f16(t.sd).reshape(12, -1)
    md = f16(t.md).reshape(12, -1)
    sq = t.sq.reshape(12, ng).astype(np.float32)
    mq = t.mq.reshape(12, ng).astype(np.float32)
    x = np.random.default_rng(nb).standard_normal(384).astype(np.float32)
    q, s, u = ob.quantize_act(x)
    y = ob.matvec(t, q, s, u)
    for r in range(12):
        c = ob.unpack(t, r).astype(np.float32).reshape(ng, 32)
        step = (sd[r][np.arange(ng) // 8] * sq[r]).astype(np.float32)
        mn = (md[r][np.arange(ng) // 8] * (mq[r] - np.float32(127))).astype(np.float32)
        want = (c * step[:, None]).astype(np.float32) + mn[:, None]
        np.testing.assert_array_equal(ob.dequant_row(t, r).reshape(ng, 32), want.astype(np.float32))
        xq = q.astype(np.float64) * np.repeat(s.astype(np.float64), 32)
        brute = float(np.dot(want.reshape(-1).astype(np.float64), xq))
        assert abs(y[r] - brute) <= 2e-6 * (np.abs(want).sum() * np.abs(xq).max() + 1e-30)


@pytest.mark.parametrize("nb", range(2, 9))
def test_plane_layout_independent_reading(tmpdir_s, nb):
    """The oracle's plane reads against a numpy reading of the layout rule
    (tooling/sml_format.py:392-448): nibble quads, 2-bit packs, 1-bit words."""
    p = tmpdir_s / f"pl{nb}.ssf"
    sa.synth_matrix(p, 4, 256, nbits=nb, seed=60 + nb)
    t = SSF(p)["w"]
    planes = t.planes()
    from sheep_amd.ssf import FLAT_PLANES
    widths = FLAT_PLANES[nb]
    for r in range(4):
        parts = []
        for w, pl in zip(widths, planes):
            if w == 4:
                b = pl.reshape(4, -1)[r].reshape(-1, 2, 32)          # quads: [half][col]
                lo, hi = b & 15, b >> 4
                g = np.stack([lo[:, 0], hi[:, 0], lo[:, 1], hi[:, 1]], 1).reshape(-1)
            elif w == 2:
                b = pl.reshape(4, -1)[r].reshape(-1, 32)
                g = np.stack([(b >> (2 * k)) & 3 for k in range(4)], 1).reshape(-1)
            else:
                b = pl.reshape(4, -1)[r]
                g = np.unpackbits(b, bitorder="little")
            parts.append(g.astype(np.int32))
        if nb == 6:
            code = parts[1] | (parts[0] << 4)
        else:
            code, sh = np.zeros(256, np.int32), 0
            for w, g in zip(widths, parts):
                code |= g << sh
                sh += w
        np.testing.assert_array_equal(ob.unpack(t, r), code.astype(np.uint8))


@needs_ref
@pytest.mark.parametrize("nb", range(2, 9))
def test_widths_match_reference(tmpdir_s, nb):
    p = tmpdir_s / f"rw{nb}.ssf"
    sa.synth_matrix(p, 64, 1536, nbits=nb, random_perm=True, seed=200 + nb)
    t = SSF(p)["w"]
    for r in (0, 17, 63):
        np.testing.assert_array_equal(ob.dequant_row(t, r), ob.ref_dequant_row(t, r))
    x = np.random.default_rng(nb).standard_normal(1536).astype(np.float32)
    q, s, u = ob.quantize_act(x)
    y, yr = ob.matvec(t, q, s, u), ob.ref_matvec(t, q, s, u)
    assert np.abs(y - yr).max() <= 1e-5 * np.abs(yr).max()


@needs_ref
@pytest.mark.parametrize("nb", [4, 8])
@pytest.mark.parametrize("cols", [128, 384, 1536, 4224])
def test_q4_q8_gemv_bit_exact_with_reference(tmpdir_s, nb, cols):
    """Q4 and Q8 rows in the reference build's lane order equal its
    sml_matvec_rows_flat4 / _flat8 bit for bit, with whole superblocks and
    with a trailing half superblock (128, 384 and 4224 columns)."""
    p = tmpdir_s / f"bx{nb}_{cols}.ssf"
    sa.synth_matrix(p, 96, cols, nbits=nb, random_perm=True, seed=cols + nb)
    t = SSF(p)["w"]
    x = (np.random.default_rng(cols).standard_normal(cols) * 3).astype(np.float32)
    q, s, u = ob.quantize_act(x[t.perm])
    y, yr = ob.matvec(t, q, s, u), ob.ref_matvec(t, q, s, u)
    np.testing.assert_array_equal(y.view(np.uint32), yr.view(np.uint32))


# ------------------------------------------------------------ small ops

def test_rms_norm_closed_form():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(1536).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(1536)).astype(np.float32)
    out = np.zeros_like(x)
    ob.oracle().orc_rms_norm(out.ctypes.data, x.ctypes.data, w.ctypes.data, 1536, 1e-6)
    ss = float(np.sum(x.astype(np.float64) ** 2))
    sc = np.float32(1) / np.sqrt(np.float32(ss / 1536) + np.float32(1e-6))
    np.testing.assert_array_equal(out, (x * sc).astype(np.float32) * w)


def test_rope_table_and_rotation():
    half, n_ctx, theta = 64, 16, 1e6
    c = np.zeros(n_ctx * half, np.float32)
    s = np.zeros(n_ctx * half, np.float32)
    ob.oracle().orc_rope_table(theta, half, n_ctx, c.ctypes.data, s.ctypes.data)
    ang = np.arange(n_ctx)[:, None] * theta ** (-np.arange(half) / half)
    assert np.abs(c.reshape(n_ctx, half) - np.cos(ang)).max() < 2e-6 * n_ctx
    assert np.abs(s.reshape(n_ctx, half) - np.sin(ang)).max() < 2e-6 * n_ctx
    x = np.random.default_rng(0).standard_normal(2 * 128).astype(np.float32)
    y = x.copy()
    ob.oracle().orc_rope(y.ctypes.data, 2, 128, half, c[5 * half:].ctypes.data, s[5 * half:].ctypes.data)
    # a rotation: each (i, i+half) pair keeps its norm
    for h in range(2):
        a, b = x[h * 128:(h + 1) * 128], y[h * 128:(h + 1) * 128]
        np.testing.assert_allclose(a[:half] ** 2 + a[half:] ** 2, b[:half] ** 2 + b[half:] ** 2, rtol=1e-5)


def test_attention_head_closed_form():
    rng = np.random.default_rng(4)
    hd, T, stride = 128, 37, 256
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal((T, stride)).astype(np.float16)
    v = rng.standard_normal((T, stride)).astype(np.float16)
    scratch = np.zeros(T, np.float32)
    out = np.zeros(hd, np.float32)
    inv = 1 / np.sqrt(np.float32(hd))
    ob.oracle().orc_attn_head(q.ctypes.data, k.view(np.uint16).ctypes.data, v.view(np.uint16).ctypes.data, stride,
                              T - 1, hd, np.float32(inv), scratch.ctypes.data, out.ctypes.data)
    sc = (k[:, :hd].astype(np.float64) @ q.astype(np.float64)) * inv
    p = np.exp(sc - sc.max())
    p /= p.sum()
    want = p @ v[:, :hd].astype(np.float64)
    np.testing.assert_allclose(out, want, rtol=1e-4, atol=1e-5)


def test_f16_roundtrip_matches_numpy():
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.standard_normal(2000) * 10.0 ** rng.uniform(-9, 5, 2000),
                         [0.0, -0.0, 65504.0, 65520.0, 1e-8, 6e-8, np.inf, -np.inf]]).astype(np.float32)
    o = ob.oracle()
    for x in xs:
        h = o.orc_f32_to_f16(float(x))
        assert h == int(np.float16(x).view(np.uint16)), x
        assert o.orc_f16_to_f32(h) == np.float32(np.float16(x)) or np.isnan(x)


def test_argmax_first_max_rule():
    """First maximum wins on ties (what np.argmax also returns); a NaN is never
    larger, so NaN at index 0 keeps 0 and NaN elsewhere is skipped."""
    rng = np.random.default_rng(6)
    o = ob.oracle()
    for n in (1, 2, 7, 1000, 151936):
        lg = rng.standard_normal(n).astype(np.float32)
        if n > 3:
            lg[n // 3] = lg[n - 1] = lg.max() + 1.0
        assert o.orc_argmax(lg.ctypes.data, n) == int(np.argmax(lg))
    lg = np.array([np.nan, 1.0, 3.0, 3.0], np.float32)
    assert o.orc_argmax(lg.ctypes.data, 4) == 0
    lg = np.array([1.0, np.nan, 3.0, 2.0], np.float32)
    assert o.orc_argmax(lg.ctypes.data, 4) == 2


def test_moe_route_golden_and_brute_force():
    g = np.load(os.path.join(GOLD, "decoder.npz"))
    lgs = g["route_lg"]
    for i in range(len(lgs)):
        sel = np.zeros(2, np.int32)
        w = np.zeros(2, np.float32)
        lg = np.ascontiguousarray(lgs[i])
        ob.oracle().orc_moe_route(lg.ctypes.data, 8, 2, 1, sel.ctypes.data, w.ctypes.data)
        np.testing.assert_array_equal(sel, g["route_sel"][i])
        np.testing.assert_array_equal(w, g["route_w"][i])
        # brute force: stable descending order (ties -> lower index), softmax over the chosen
        order = sorted(range(8), key=lambda e: (-lg[e], e))[:2]
        assert list(sel) == order
        e = np.exp(lg[order].astype(np.float64) - lg[order[0]])
        np.testing.assert_allclose(w, e / e.sum(), rtol=1e-6)


# ------------------------------------------------------------ decoder

def test_decoder_golden(tmpdir_s):
    """The oracle's decoder equals, bit for bit, the logits the reference's
    sml_forward wrote for a zero-mean synthetic decoder, greedy from token 5."""
    g = np.load(os.path.join(GOLD, "decoder.npz"))
    p = tmpdir_s / "tiny.ssf"
    sa.synth_model(p, n_layer=2, n_embd=256, n_head=2, n_head_kv=1, n_ff=512, n_vocab=1000,
                   qkv_bias=True, random_perm=True, seed=7)
    assert hashlib.sha256(p.read_bytes()).digest() == g["sha"].tobytes()
    m = ob.OracleModel(p, 32)
    toks = g["tokens"]
    assert len(set(toks.tolist())) >= 8, "the golden decoder's greedy ids are not diverse"
    for pos in range(len(toks) - 1):
        lg = m.forward(int(toks[pos]), pos)
        np.testing.assert_array_equal(lg.view(np.uint32), g["logits"][pos].view(np.uint32), err_msg=f"position {pos}")
        assert int(np.argmax(lg)) == int(toks[pos + 1])
    m.close()


def test_zero_mean_decoder_is_informative(tmpdir_s):
    """The synthetic decoders' weights have mean zero (mins at -(2^b-1)/2 steps),
    so the logits depend on the input. Teacher-forced on random ids, the part
    of the logits' variance that changes from position to position is a fifth
    of the whole and the argmax moves; with the single-GEMV recipe (mins at
    -2^(b-1) steps) a common term carries over 97% of the variance and the
    argmax barely moves."""
    rng = np.random.default_rng(11)
    ids = rng.integers(0, 2000, 24)
    for zero_mean in (True, False):
        p = tmpdir_s / f"inf{int(zero_mean)}.ssf"
        sa.synth_model(p, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000,
                       qkv_bias=True, random_perm=True, seed=31, zero_mean=zero_mean)
        m = ob.OracleModel(p, 32)
        L = np.stack([m.forward(int(t), i) for i, t in enumerate(ids)]).astype(np.float64)
        m.close()
        distinct = len(set(np.argmax(L, 1).tolist()))
        frac = (L - L.mean(0)).var() / L.var()
        if zero_mean:
            assert frac > 0.1 and distinct >= 4, (frac, distinct)
        else:
            assert frac < 0.03 and distinct <= 2, (frac, distinct)


def test_expf_restatement_equals_the_library():
    """The restated expf (the GPU's exact softmax and routing weights use the
    same algorithm and table) equals the C library's expf bit for bit on
    every 7th float from -0.0 down to -inf and from +0.0 up to +inf (613 M
    inputs: normals, denormals, the underflow edge at -103.97, the overflow
    edge at 88.72, the infinities), and on the closed forms."""
    o = ob.oracle()
    assert o.orc_expf_mismatches(7) == 0
    assert o.orc_expf_published(0.0) == 1.0
    assert o.orc_expf_published(-200.0) == 0.0
    assert o.orc_expf_published(89.0) == np.inf
    assert o.orc_expf_published(88.7) == np.float32(np.exp(np.float64(np.float32(88.7))))
    for x in (-1.0, -0.5, -10.0, -50.3):        # correctly rounded from double here
        assert o.orc_expf_published(x) == float(np.float32(np.exp(np.float64(np.float32(x))))), x


def test_silu_polynomial_closed_form():
    """The SwiGLU activation with the reference build's 2^x polynomial
    (sml/sml-run.c:393-426): within 2.5e-4 relative of g/(1+e^-g)*u in float64
    over the range the FFN sees (the polynomial's own ~1.5e-4, as the
    reference documents it at :466-469), and exactly g*u where the exponent
    clamps. The decoder tests pin it bit for bit against the reference build."""
    rng = np.random.default_rng(12)
    g = np.concatenate([rng.standard_normal(4000) * 4, rng.uniform(-30, 30, 4000), [0.0, 1e-30, 87.0, 95.0]]).astype(np.float32)
    u = rng.standard_normal(len(g)).astype(np.float32)
    out = g.copy()
    ob.oracle().orc_silu_mul(out.ctypes.data, u.ctypes.data, len(g))
    g64 = g.astype(np.float64)
    want = g64 / (1 + np.exp(-g64)) * u.astype(np.float64)
    assert (np.abs(out - want) <= 2.5e-4 * np.abs(want) + 1e-30).all()
    assert out[-1] == g[-1] * u[-1]


@needs_ref
@pytest.mark.parametrize("model", ["dense", "moe", "qwen_layer"])
def test_decoder_bit_exact_with_reference(tmpdir_s, model):
    """The oracle's whole decode step against the reference's own sml_forward,
    teacher-forced on 32 random ids: every logit equal bit for bit (GEMV lane
    order and FMAs, attention chains, softmax, SiLU polynomial, RoPE, norms,
    router and expert sums), and the reference's argmax takes many values."""
    cfg = {
        "dense": dict(n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000, qkv_bias=True,
                      random_perm=True, seed=31),
        "moe": dict(n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=600, n_expert=4,
                    n_expert_used=2, moe_flags=1, random_perm=True, seed=5),
        "qwen_layer": dict(n_layer=1, n_embd=1536, n_head=12, n_head_kv=2, n_ff=8960, n_vocab=4000,
                           rope_theta=1e6, qkv_bias=True, tied=True, random_perm=True, seed=1002),
    }[model]
    p = tmpdir_s / f"bx_{model}.ssf"
    sa.synth_model(p, **cfg)
    ids = np.random.default_rng(3).integers(0, cfg["n_vocab"], 32)
    om, rm = ob.OracleModel(p, 64), ob.RefModel(p, 64, threads=4)
    arg = []
    try:
        for pos, tok in enumerate(ids):
            a, b = om.forward(int(tok), pos), rm.forward(int(tok), pos)
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"position {pos}")
            arg.append(int(np.argmax(b)))
    finally:
        om.close()
        rm.close()
    assert len(set(arg)) >= 8, arg


@needs_ref
@pytest.mark.parametrize("perm", [False, True])
def test_moe_decoder_matches_reference(tmpdir_s, perm):
    """A Mixtral-shaped decoder (4 experts, top-2, softmax over the chosen):
    the oracle's router, routing and expert FFN against the reference's
    sml_forward, position by position."""
    p = tmpdir_s / f"moe_dec_{int(perm)}.ssf"
    sa.synth_model(p, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=600, n_expert=4,
                   n_expert_used=2, moe_flags=1, random_perm=perm, seed=55 + int(perm))
    om, rm = ob.OracleModel(p, 16), ob.RefModel(p, 16, threads=1)
    try:
        for pos, tok in enumerate([1, 77, 300, 5, 599, 42]):
            a, b = om.forward(tok, pos), rm.forward(tok, pos)
            np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32), err_msg=f"position {pos}")
    finally:
        om.close()
        rm.close()


@needs_ref
def test_per256_regime_matches_reference_multi(tmpdir_s, monkeypatch):
    """The oracle's per-256 regime (every product's input quantized by
    sml_quantize_act_sb, then the per-group kernels) against the reference's
    sml_forward_multi in its default regime for four sequences
    (sml/sml-run.c:2559-2599), teacher-forced on the reference's tokens.
    Float orders differ, so an int8 code flips now and then (one flip at the
    head moves the logits ~1e-3): the mean distance must stay under a third
    of the reference's own per-32 stepping's distance to the same logits."""
    monkeypatch.delenv("SML_MULTI", raising=False)
    monkeypatch.delenv("SML_MULTI_EXACT_MAX", raising=False)
    p = tmpdir_s / "per256.ssf"
    sa.synth_model(p, n_layer=1, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000, qkv_bias=True,
                   random_perm=True, seed=74)
    prompts = [[5, 17, 300], [1], [42, 42, 7, 1999, 3], [250, 11]]
    m, alone = ob.RefMulti(p, 64, 4, threads=2), ob.RefMulti(p, 64, 4, threads=2)
    oms = [ob.OracleModel(p, 64) for _ in prompts]
    rd = lambda a, b: np.sqrt(((a - b) ** 2).mean() / (b ** 2).mean())
    d_orc, d_regime = [], []
    try:
        toks, pos = [], []
        for b, pr in enumerate(prompts):
            for i, t in enumerate(pr):
                lr = m.forward(b, t, i)
                alone.forward(b, t, i)
                oms[b].forward(t, i)
            toks.append(int(np.argmax(lr)))
            pos.append(len(pr))
        for o in oms:
            o.per256(True)
        for _ in range(6):
            ref = m.step(toks, pos).astype(np.float64)
            orc = np.stack([oms[b].forward(toks[b], pos[b]) for b in range(4)]).astype(np.float64)
            ex = np.stack([alone.forward(b, toks[b], pos[b]) for b in range(4)]).astype(np.float64)
            d_orc.append(rd(orc, ref))
            d_regime.append(rd(ex, ref))
            toks = [int(np.argmax(r)) for r in ref]
            pos = [q + 1 for q in pos]
    finally:
        m.close()
        alone.close()
        for o in oms:
            o.close()
    assert np.mean(d_regime) > 1e-3                   # the regimes are told apart at all
    assert np.mean(d_orc) < np.mean(d_regime) / 3, (np.mean(d_orc), np.mean(d_regime))


# ------------------------------------------------------------ GPTQ-style 4-bit

def test_gptq_packing_bit_order():
    """The documented AutoGPTQ layout (tooling/sml_unpack.py:66-76): input 8k+i
    of output o in bits 4i..4i+3 of qweight[k, o]; output 8j+i's zero in bits
    4i..4i+3 of qzeros[g, j]; v1 stores zero - 1."""
    from sheep_amd import gptq as gq
    codes = np.zeros((8, 128), np.uint8)
    codes[0, :8] = np.arange(8)
    zeros = np.arange(1, 9).reshape(8, 1)
    qw, qz, _ = gq.pack(codes, zeros, np.ones((8, 1)), zero_add=1)
    assert qw.view(np.uint32)[0, 0] == 0x76543210 and not qw.view(np.uint32)[1:, 0].any()
    assert qz.view(np.uint32)[0, 0] == 0x76543210
    c, z = ob.gptq_unpack_row(qw, qz, 8, 128, 0)
    assert list(c[:8]) == list(range(8)) and not c[8:].any() and z[0] == 1


@pytest.mark.parametrize("zero_add", [1, 0])
def test_gptq_known_answer(zero_add):
    """The known answer of mlmi/tests/test_unpack.py:74-103 restated: 64 inputs x
    32 outputs, group 16, codes 0..15, zeros 1..15, fp16 scales in [0.1, 1.1);
    unpacking the packed arrays gives (q - z) * s exactly (max |diff| 0.0)."""
    from sheep_amd import gptq as gq
    rng = np.random.default_rng(0)
    IN, OUT, GS = 64, 32, 16
    q = rng.integers(0, 16, (OUT, IN))
    z = rng.integers(1, 16, (OUT, IN // GS))
    s = (rng.random((OUT, IN // GS)) + 0.1).astype(np.float16)
    qw, qz, sc = gq.pack(q, z, s, zero_add=zero_add)
    W = np.zeros((OUT, IN), np.float32)
    for o in range(OUT):
        c, zz = ob.gptq_unpack_row(qw, qz, OUT, IN, o, group=GS, zero_add=zero_add)
        np.testing.assert_array_equal(c, q[o])
        np.testing.assert_array_equal(zz, z[o])
        W[o] = ob.gptq_dequant_row(qw, qz, sc, OUT, IN, o, group=GS, zero_add=zero_add)
    want = (q - np.repeat(z, GS, axis=1)).astype(np.float32) * np.repeat(s.astype(np.float32), GS, axis=1)
    assert np.abs(W - want).max() == 0.0
    x = rng.standard_normal(IN).astype(np.float32)
    y = ob.gptq_matvec(qw, qz, sc, OUT, IN, x, group=GS, zero_add=zero_add)
    np.testing.assert_allclose(y, (want.astype(np.float64) @ x.astype(np.float64)).astype(np.float32), rtol=1e-6, atol=1e-6)


def test_gptq_desc_act_closed_form():
    """desc_act (dequant_gptq's g_idx branch, tooling/sml_unpack.py:90-96):
    input k takes the zero and scale of group g_idx[k]. On the known answer's
    shapes with a scattered g_idx: every weight is (q - z[g_idx[k]]) * s[g_idx[k]]
    exactly, and an identity g_idx equals the plain reading bit for bit."""
    from sheep_amd import gptq as gq
    rng = np.random.default_rng(1)
    IN, OUT, GS = 64, 32, 16
    q = rng.integers(0, 16, (OUT, IN))
    zg = rng.integers(1, 16, (OUT, IN // GS))
    s = (rng.random((OUT, IN // GS)) + 0.1).astype(np.float16)
    g_idx = gq.desc_act_gidx(IN, 3, group=GS)
    assert sorted(np.bincount(g_idx).tolist()) == [GS] * (IN // GS) and (g_idx != np.arange(IN) // GS).any()
    qw, qz, sc = gq.pack(q, zg, s, zero_add=1)
    for o in range(OUT):
        w = ob.gptq_dequant_row_gidx(qw, qz, sc, g_idx, OUT, IN, o, group=GS)
        want = (q[o] - zg[o][g_idx]).astype(np.float32) * s[o][g_idx].astype(np.float32)
        assert np.abs(w - want).max() == 0.0
        ident = ob.gptq_dequant_row_gidx(qw, qz, sc, (np.arange(IN) // GS).astype(np.int32), OUT, IN, o, group=GS)
        np.testing.assert_array_equal(ident, ob.gptq_dequant_row(qw, qz, sc, OUT, IN, o, group=GS))


@pytest.mark.parametrize("with_zeros", [True, False])
def test_awq_known_answer(with_zeros):
    """The AWQ half of mlmi/tests/test_unpack.py:74-103 restated: 64 inputs x
    32 outputs, group 16, words packed along the output with the test's own
    order (nibble i holds output (0, 2, 4, 6, 1, 3, 5, 7)[i] of its 8), zeros
    stored as they are (without qzeros: 8). Reading them back gives
    (q - z) * s exactly, and the repo's packer writes the same words."""
    from sheep_amd import gptq as gq
    rng = np.random.default_rng(1)
    IN, OUT, GS = 64, 32, 16
    q = rng.integers(0, 16, (IN, OUT)).astype(np.uint32)
    z = rng.integers(1, 16, (IN // GS, OUT)).astype(np.uint32) if with_zeros else np.full((IN // GS, OUT), 8, np.uint32)
    s = (rng.random((IN // GS, OUT)) + 0.1).astype(np.float16)
    order = (0, 2, 4, 6, 1, 3, 5, 7)

    def pack(x):                               # [r, OUT] -> [r, OUT/8]
        x = x.reshape(x.shape[0], -1, 8)[:, :, list(order)]
        return sum(x[:, :, i] << np.uint32(4 * i) for i in range(8)).astype(np.uint32).view(np.int32)

    qw, qz = pack(q), (pack(z) if with_zeros else None)
    sc = np.ascontiguousarray(s)
    want = (q.astype(np.int64) - np.repeat(z, GS, axis=0)).astype(np.float32).T * \
        np.repeat(s.astype(np.float32), GS, axis=0).T
    for o in range(OUT):
        c, zz = ob.awq_unpack_row(qw, qz, OUT, IN, o, group=GS)
        np.testing.assert_array_equal(c, q[:, o])
        np.testing.assert_array_equal(zz, z[:, o])
        w = ob.awq_dequant_row(qw, qz, sc, OUT, IN, o, group=GS)
        assert np.abs(w - want[o]).max() == 0.0
    pw, pz, ps = gq.pack_awq(q.T, z.T if with_zeros else None, s.T)
    np.testing.assert_array_equal(pw, qw)
    if with_zeros:
        np.testing.assert_array_equal(pz, qz)
    np.testing.assert_array_equal(ps, sc)


ROUTE_MODES = [   # (moe_flags, scale, groups, topk_group, bias)
    (0, 0.0, 1, 1, False), (1, 0.0, 1, 1, False), (0, 1.5, 1, 1, False),        # plain top-k; DeepSeek V2 greedy
    (2, 0.0, 1, 1, True), (3, 2.5, 8, 4, True), (3, 2.5, 8, 3, False),         # sigmoid + bias (V3 noaux_tc)
    (1, 0.0, 4, 2, False), (9, 1.0, 4, 1, False), (0, 0.0, 1, 1, True),        # softmax scores, groups, bias
    (4, 0.01, 1, 1, False), (4, 0.1, 1, 1, False),                             # PhiMoE sparsemixer
]


@needs_ref
@pytest.mark.parametrize("mode", ROUTE_MODES)
def test_moe_route_every_mode_equals_the_reference(mode):
    """orc_moe_route2 against the reference's own sml_moe_route (through the
    shim, on a header and layer holding the routing fields) on 400 logit
    vectors per mode, 64 and 16 experts: the same choices and the same
    weights bit for bit, including ties (logits rounded to a coarse grid)."""
    flags, scale, groups, tg, bias = mode
    rng = np.random.default_rng(flags * 100 + groups)
    for ne, k in ((64, 8), (16, 4)):
        g = groups if ne % groups == 0 else 1
        for i in range(400):
            lg = (rng.standard_normal(ne) * 2).astype(np.float32)
            if i % 4 == 1:
                lg = (np.round(lg * 4) / 4).astype(np.float32)      # ties
            eb = (rng.standard_normal(ne) * 0.1).astype(np.float32) if bias else None
            out = []
            for fn in (ob.oracle().orc_moe_route2, ob.ref().ref_moe_route2):
                sel, w = np.zeros(k, np.int32), np.zeros(k, np.float32)
                assert fn(lg.ctypes.data, ne, k, flags, scale, g, tg, eb.ctypes.data if bias else None,
                          sel.ctypes.data, w.ctypes.data) == k
                out.append((sel, w))
            np.testing.assert_array_equal(out[0][0], out[1][0], err_msg=f"{mode} {ne} #{i} choices")
            np.testing.assert_array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32),
                                          err_msg=f"{mode} {ne} #{i} weights")
