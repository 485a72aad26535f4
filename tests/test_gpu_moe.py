"""Small-M GEMM and the MoE expert FFN on the GPU against the oracle.

The small-M GEMM streams each weight once for all its rows with the GEMV's
per-row arithmetic order, so each row's output equals the GEMV's exactly.
MoE routing (the chosen experts) must equal the oracle's restatement of
sml_moe_route bit for bit; logits and weights agree to float rounding of the
same double sums; the FFN output is within 1e-3 of the oracle's per-token
composition (quantize, gate/up, SiLU, quantize, down, weighted sum in choice
order).
"""
import numpy as np
import pytest

import sheep_amd as sa
from oracle import bind as ob
from sheep_amd.ssf import SSF

pytestmark = pytest.mark.gpu

TOL_MAX = 1e-3
TOL_RMS = 1e-4


@pytest.fixture(scope="module", autouse=True)
def device():
    sa.init(0)


def close(gpu, ref, what):
    err = np.abs(gpu.astype(np.float64) - ref.astype(np.float64))
    scale = np.abs(ref).max()
    rms = np.sqrt((err ** 2).mean()) / max(np.sqrt((ref.astype(np.float64) ** 2).mean()), 1e-30)
    assert err.max() <= TOL_MAX * scale, f"{what}: max err {err.max():.3g} vs scale {scale:.3g}"
    assert rms <= TOL_RMS, f"{what}: rel-RMS {rms:.3g}"


def quant_rows(xs):
    q, s, u = zip(*(ob.quantize_act(np.ascontiguousarray(x, np.float32)) for x in xs))
    return (sa.DevBuf.of(np.concatenate(q)), sa.DevBuf.of(np.concatenate(s)), sa.DevBuf.of(np.concatenate(u)))


@pytest.mark.parametrize("nb", [4, 3, 6, 8])
@pytest.mark.parametrize("cols", [1536, 5120])
def test_gemm_rows_equal_gemv(tmpdir_s, nb, cols, monkeypatch):
    """The exact regime (SML_MULTI=exact): each row bit for bit the GEMV's."""
    monkeypatch.setenv("SML_MULTI", "exact")
    p = tmpdir_s / f"gemm{nb}_{cols}.ssf"
    if not p.exists():
        sa.synth_matrix(p, 1000, cols, nbits=nb, random_perm=False, seed=300 + nb)
    t = SSF(p)["w"]
    m = sa.Mat.from_file(p, "w")
    rng = np.random.default_rng(nb * cols)
    for nrow in (1, 3, 4, 7, 16):
        xs = [rng.standard_normal(cols).astype(np.float32) * (1 + r) for r in range(nrow)]
        q, s, u = quant_rows(xs)
        y = sa.DevBuf(nrow * 1000 * 4)
        sa.gemm(m, q, s, u, nrow, y)
        got = y.read(np.float32).reshape(nrow, 1000)
        for r in range(nrow):
            act = sa.Act(cols)
            act.q.write(ob.quantize_act(xs[r])[0]); act.scale.write(ob.quantize_act(xs[r])[1])
            act.sums.write(ob.quantize_act(xs[r])[2])
            y1 = sa.DevBuf(1000 * 4)
            sa.matvec(m, act, y1)
            np.testing.assert_array_equal(got[r], y1.read(np.float32), err_msg=f"row {r} of {nrow}")
            close(got[r], ob.matvec(t, *ob.quantize_act(xs[r])), f"gemm q{nb} row {r}")


@pytest.mark.parametrize("cols,rows", [(1536, 1000), (5120, 2048), (4096, 40000)])
def test_mfma_gemm_q4(tmpdir_s, cols, rows):
    """Q4 with more than 8 rows on MFMA: each row within 1e-3 of the oracle."""
    p = tmpdir_s / f"mg_{cols}_{rows}.ssf"
    if not p.exists():
        sa.synth_matrix(p, rows, cols, nbits=4, random_perm=False, seed=400 + cols)
    t = SSF(p)["w"]
    m = sa.Mat.from_file(p, "w")
    rng = np.random.default_rng(cols)
    for nrow in (9, 16):
        xs = [rng.standard_normal(cols).astype(np.float32) * (1 + r) for r in range(nrow)]
        q, s, u = quant_rows(xs)
        y = sa.DevBuf(nrow * rows * 4)
        sa.gemm(m, q, s, u, nrow, y)
        got = y.read(np.float32).reshape(nrow, rows)
        for r in range(nrow):
            close(got[r], ob.matvec(t, *ob.quantize_act(xs[r])), f"mfma gemm row {r} of {nrow}")


@pytest.mark.parametrize("cols", [1536, 4096])
def test_mfma_gemm_persistent_equals_one_tile(tmpdir_s, monkeypatch, cols):
    """The persistent MFMA GEMM (a workgroup walks several 16-row tiles with
    its activation operands kept in registers) computes each tile with the
    one-tile kernel's arithmetic: outputs equal bit for bit, whatever the grid
    (the default cap, 5 workgroups for 563 tiles, one tile each), for plain
    and SwiGLU products, per-32 and per-256 activations; the last tile is
    ragged (9000 rows)."""
    rows = 9000
    p = tmpdir_s / f"mgp_{cols}.ssf"
    if not p.exists():
        sa.synth_matrix(p, rows, cols, nbits=4, random_perm=False, seed=700 + cols)
    m = sa.Mat.from_file(p, "w")
    up = sa.Mat.from_file(p, "w")
    rng = np.random.default_rng(cols + 7)
    nrow = 13
    xs = [rng.standard_normal(cols).astype(np.float32) * (1 + r) for r in range(nrow)]
    for per256 in (False, True):
        q, s, u = quant_rows_sb(xs) if per256 else (None, None, None)
        acts = (sa.DevBuf.of(q), sa.DevBuf.of(s), sa.DevBuf.of(u)) if per256 else quant_rows(xs)
        outs = {}
        for mode, env in (("one tile", {"SML_MGEMM_PS": "0"}), ("default", {}), ("5 workgroups", {"SML_MGEMM_PWG": "5"})):
            monkeypatch.delenv("SML_MGEMM_PS", raising=False)
            monkeypatch.delenv("SML_MGEMM_PWG", raising=False)
            for k, v in env.items():
                monkeypatch.setenv(k, v)
            y = sa.DevBuf(nrow * rows * 4)
            sa.gemm(m, *acts, nrow, y, per256=per256)
            h = sa.DevBuf(nrow * rows * 4)
            sa.gemm_swiglu(m, up, *acts, nrow, h, per256=per256)
            outs[mode] = (y.read(np.float32), h.read(np.float32))
        for mode in ("default", "5 workgroups"):
            for i, what in enumerate(("plain", "swiglu")):
                np.testing.assert_array_equal(outs[mode][i], outs["one tile"][i],
                                              err_msg=f"{what} per256={per256} {mode}")
        assert np.isfinite(outs["one tile"][0]).all()


@pytest.mark.parametrize("cols,rows", [(5120, 2048), (14336, 1000)])
def test_mfma_gemm_split_k_close_to_one_pass(tmpdir_s, monkeypatch, cols, rows):
    """Inputs wider than 16 superblocks split into 4 slices (a persistent
    workgroup per slice and row tiles, then sml_gemm_ksum adds the slices in
    order): every output within float rounding of the one-pass kernel
    (SML_MGEMM_KS=1), which sums each wave's superblocks and then the waves
    in another order; per-32 and per-256 activations, 9 and 16 rows, a
    ragged last tile (1000 rows)."""
    p = tmpdir_s / f"mgk_{cols}_{rows}.ssf"
    if not p.exists():
        sa.synth_matrix(p, rows, cols, nbits=4, random_perm=False, seed=900 + cols)
    m = sa.Mat.from_file(p, "w")
    rng = np.random.default_rng(cols + 9)
    for nrow in (9, 16):
        xs = [rng.standard_normal(cols).astype(np.float32) * (1 + r) for r in range(nrow)]
        for per256 in (False, True):
            acts = tuple(sa.DevBuf.of(a) for a in quant_rows_sb(xs)) if per256 else quant_rows(xs)
            outs = {}
            for ks in ("1", "4"):
                monkeypatch.setenv("SML_MGEMM_KS", ks)
                y = sa.DevBuf(nrow * rows * 4)
                sa.gemm(m, *acts, nrow, y, per256=per256)
                outs[ks] = y.read(np.float32).reshape(nrow, rows)
            a, b = outs["4"], outs["1"]
            assert np.isfinite(a).all()
            scale = np.abs(b).max(axis=1, keepdims=True)
            err = float((np.abs(a - b) / scale).max())
            assert err < 1e-5, (nrow, per256, err)
            assert not np.array_equal(a, b), "the split form did not run"


def quant_rows_sb(xs):
    """Per-256 quantization of each row (sml_quantize_act_sb), as host arrays."""
    q, s, u = zip(*(ob.quantize_act(np.ascontiguousarray(x, np.float32), per256=True) for x in xs))
    return np.stack(q), np.stack(s), np.stack(u)


@pytest.mark.skipif(not ob.have_ref(), reason="oracle/_ref (the reference's CPU engine) is not built")
@pytest.mark.parametrize("cols,rows", [(1536, 1000), (5120, 2048), (14336, 4096)])
def test_gemm_q4_per256_matches_reference(tmpdir_s, cols, rows):
    """Per-256 activations (the batched regime) on MFMA with integer
    superblock sums: every row within 1e-3 of the reference's
    sml_matvec_batch_flat4_sb and of its once-packed rows-in-lanes
    sml_rlp_matvec, for 1 to 16 rows."""
    p = tmpdir_s / f"mgsb_{cols}_{rows}.ssf"
    if not p.exists():
        sa.synth_matrix(p, rows, cols, nbits=4, random_perm=False, seed=500 + cols)
    t = SSF(p)["w"]
    m = sa.Mat.from_file(p, "w")
    rng = np.random.default_rng(cols + 1)
    for nrow in (1, 3, 4, 9, 16):
        xs = [rng.standard_normal(cols).astype(np.float32) * (1 + r) for r in range(nrow)]
        Q, S, U = quant_rows_sb(xs)
        y = sa.DevBuf(nrow * rows * 4)
        sa.gemm(m, sa.DevBuf.of(Q), sa.DevBuf.of(S), sa.DevBuf.of(U), nrow, y, per256=True)
        got = y.read(np.float32).reshape(nrow, rows)
        want = ob.ref_matvec_batch(t, Q, S, U, sb=True)
        rlp = ob.ref_rlp_matvec(t, Q, S, U)
        assert rlp is not None
        for r in range(nrow):
            close(got[r], want[r], f"per-256 gemm row {r} of {nrow} vs flat4_sb")
            close(got[r], rlp[r], f"per-256 gemm row {r} of {nrow} vs rlp")


@pytest.mark.parametrize("nb", [2, 3, 5, 6, 8])
def test_gemm_per256_other_widths(tmpdir_s, nb):
    """Widths other than Q4 take per-256 activations through the per-group
    kernels, on which the reference's own kernels are exact (the scale
    repeats in every group, sml/sml-kernel.h:314-318): each row within 1e-3
    of the reference's decode kernel on the same activation."""
    if not ob.have_ref():
        pytest.skip("oracle/_ref (the reference's CPU engine) is not built")
    cols, rows = 2048, 1000
    p = tmpdir_s / f"gsb{nb}.ssf"
    if not p.exists():
        sa.synth_matrix(p, rows, cols, nbits=nb, random_perm=False, seed=600 + nb)
    t = SSF(p)["w"]
    m = sa.Mat.from_file(p, "w")
    rng = np.random.default_rng(nb)
    xs = [rng.standard_normal(cols).astype(np.float32) for _ in range(5)]
    Q, S, U = quant_rows_sb(xs)
    y = sa.DevBuf(5 * rows * 4)
    sa.gemm(m, sa.DevBuf.of(Q), sa.DevBuf.of(S), sa.DevBuf.of(U), 5, y, per256=True)
    got = y.read(np.float32).reshape(5, rows)
    for r in range(5):
        close(got[r], ob.ref_matvec(t, Q[r], S[r], U[r]), f"q{nb} per-256 row {r}")


@pytest.mark.skipif(not ob.have_ref(), reason="oracle/_ref (the reference's CPU engine) is not built")
def test_gemm_swiglu_per256(tmpdir_s):
    p = tmpdir_s / "gemm_ffn_sb.ssf"
    sa.synth_model(p, n_layer=1, n_embd=1536, n_head=12, n_head_kv=2, n_ff=2048, n_vocab=256, seed=42)
    f = SSF(p)
    g, u = f["blk.0.ffn_gate.weight"], f["blk.0.ffn_up.weight"]
    mg, mu = sa.Mat.from_file(p, g.name), sa.Mat.from_file(p, u.name)
    rng = np.random.default_rng(6)
    xs = [rng.standard_normal(1536).astype(np.float32)[g.perm] for _ in range(12)]
    Q, S, U = quant_rows_sb(xs)
    h = sa.DevBuf(12 * 2048 * 4)
    sa.gemm_swiglu(mg, mu, sa.DevBuf.of(Q), sa.DevBuf.of(S), sa.DevBuf.of(U), 12, h, per256=True)
    got = h.read(np.float32).reshape(12, 2048)
    yg, yu = ob.ref_matvec_batch(g, Q, S, U, sb=True), ob.ref_matvec_batch(u, Q, S, U, sb=True)
    for r in range(12):
        ob.oracle().orc_silu_mul(yg[r].ctypes.data, yu[r].ctypes.data, 2048)
        close(got[r], yg[r], f"per-256 gemm swiglu row {r}")


def test_gemm_swiglu_rows(tmpdir_s):
    p = tmpdir_s / "gemm_ffn.ssf"
    sa.synth_model(p, n_layer=1, n_embd=1536, n_head=12, n_head_kv=2, n_ff=2048, n_vocab=256, seed=41)
    f = SSF(p)
    g, u = f["blk.0.ffn_gate.weight"], f["blk.0.ffn_up.weight"]
    mg, mu = sa.Mat.from_file(p, g.name), sa.Mat.from_file(p, u.name)
    rng = np.random.default_rng(5)
    xs = [rng.standard_normal(1536).astype(np.float32) for _ in range(5)]
    q, s, su = quant_rows([x[g.perm] for x in xs])
    h = sa.DevBuf(5 * 2048 * 4)
    sa.gemm_swiglu(mg, mu, q, s, su, 5, h)
    got = h.read(np.float32).reshape(5, 2048)
    for r, x in enumerate(xs):
        qa, sa_, ua = ob.quantize_act(x[g.perm])
        yg, yu = ob.matvec(g, qa, sa_, ua), ob.matvec(u, qa, sa_, ua)
        ob.oracle().orc_silu_mul(yg.ctypes.data, yu.ctypes.data, 2048)
        close(got[r], yg, f"gemm swiglu row {r}")


def moe_model(tmpdir_s, name, n_embd, n_ff, nexp, k, perm, seed):
    p = tmpdir_s / name
    if not p.exists():
        sa.synth_model(p, n_layer=1, n_embd=n_embd, n_head=n_embd // 128, n_head_kv=2, n_ff=n_ff, n_vocab=512,
                       n_expert=nexp, n_expert_used=k, moe_flags=1, random_perm=perm, seed=seed)
    return p


def oracle_moe(f, x, nexp, k, n_embd, flags=1, per256=False):
    """Per token, as moe_ffn (sml/sml-run.c:3071-3124) with the oracle's
    kernels; per256 quantizes the expert inputs as moe_ffn_batch does in the
    batched regimes."""
    router = np.ascontiguousarray(f["blk.0.ffn_gate_inp.weight"].f32)
    lg = np.zeros(nexp, np.float32)
    ob.oracle().orc_router(router.ctypes.data, x.ctypes.data, nexp, n_embd, lg.ctypes.data)
    sel = np.zeros(k, np.int32)
    w = np.zeros(k, np.float32)
    ob.oracle().orc_moe_route(lg.ctypes.data, nexp, k, flags, sel.ctypes.data, w.ctypes.data)
    acc = np.zeros(n_embd, np.float32)
    for j in range(k):
        e = int(sel[j])
        g, u, d = (f[f"blk.0.ffn_{kind}.{e}.weight"] for kind in ("gate", "up", "down"))
        qa = ob.quantize_act(np.ascontiguousarray(x[g.perm]), per256)
        yg, yu = ob.matvec(g, *qa), ob.matvec(u, *qa)
        ob.oracle().orc_silu_mul(yg.ctypes.data, yu.ctypes.data, len(yg))
        yd = ob.matvec(d, *ob.quantize_act(np.ascontiguousarray(yg[d.perm]), per256))
        acc += w[j] * yd
    return lg, sel, w, acc


@pytest.mark.parametrize("T,perm", [(1, False), (5, True), (16, False), (16, True)])
def test_moe_ffn(tmpdir_s, T, perm):
    n_embd, n_ff, nexp, k = 1024, 1536, 8, 2
    p = moe_model(tmpdir_s, f"moe_{int(perm)}.ssf", n_embd, n_ff, nexp, k, perm, seed=1005 + int(perm))
    f = SSF(p)
    moe = sa.MoE(p, 0, 16)
    assert (moe.nexp, moe.k, moe.n_ff) == (nexp, k, n_ff)
    rng = np.random.default_rng(T * 7 + int(perm))
    x = rng.standard_normal((T, n_embd)).astype(np.float32)
    out, sel, w, lg = sa.DevBuf(T * n_embd * 4), sa.DevBuf(T * k * 4), sa.DevBuf(T * k * 4), sa.DevBuf(T * nexp * 4)
    moe.ffn(sa.DevBuf.of(x), T, out, sel, w, lg)
    got_out = out.read(np.float32).reshape(T, n_embd)
    got_sel = sel.read(np.int32).reshape(T, k)
    got_w = w.read(np.float32).reshape(T, k)
    got_lg = lg.read(np.float32).reshape(T, nexp)
    for t in range(T):
        rl, rs, rw, ro = oracle_moe(f, x[t], nexp, k, n_embd)
        np.testing.assert_allclose(got_lg[t], rl, rtol=1e-6, atol=1e-7)
        np.testing.assert_array_equal(got_sel[t], rs, err_msg=f"token {t} routing")
        np.testing.assert_allclose(got_w[t], rw, rtol=1e-6, atol=1e-7)
        close(got_out[t], ro, f"moe token {t}")


@pytest.mark.parametrize("T", [4, 16])
def test_moe_ffn_per256(tmpdir_s, T):
    """The batched regime's expert products: inputs quantized per 256
    (bit-exact routing still), each token's output within 1e-3 of the
    oracle's per-token composition on per-256 activations."""
    n_embd, n_ff, nexp, k = 1024, 1536, 8, 2
    p = moe_model(tmpdir_s, "moe_1.ssf", n_embd, n_ff, nexp, k, True, seed=1006)
    f = SSF(p)
    moe = sa.MoE(p, 0, 16)
    moe.regime(True)
    rng = np.random.default_rng(T * 11)
    x = rng.standard_normal((T, n_embd)).astype(np.float32)
    out, sel = sa.DevBuf(T * n_embd * 4), sa.DevBuf(T * k * 4)
    moe.ffn(sa.DevBuf.of(x), T, out, sel)
    got_out = out.read(np.float32).reshape(T, n_embd)
    got_sel = sel.read(np.int32).reshape(T, k)
    for t in range(T):
        _, rs, _, ro = oracle_moe(f, x[t], nexp, k, n_embd, per256=True)
        np.testing.assert_array_equal(got_sel[t], rs, err_msg=f"token {t} routing")
        close(got_out[t], ro, f"per-256 moe token {t}")


@pytest.mark.parametrize("per256", [False, True])
def test_moe_expert_with_many_tokens(tmpdir_s, per256, monkeypatch):
    """An expert chosen by more than 8 of 16 tokens goes to the second size
    class's launch (up to 16 rows): 12 identical tokens send 12 rows to the
    same two experts. Routing is bit-exact and every token's output close
    to the oracle's; with SML_GEMM_SPLIT=0 (one launch of the 16-row class
    for every group) the outputs are the same bits."""
    n_embd, n_ff, nexp, k, T = 1024, 1536, 8, 2, 16
    p = moe_model(tmpdir_s, "moe_0.ssf", n_embd, n_ff, nexp, k, False, seed=1005)
    f = SSF(p)
    rng = np.random.default_rng(91)
    x = rng.standard_normal((T, n_embd)).astype(np.float32)
    x[1:12] = x[0]
    outs = {}
    for split in ("1", "0"):
        monkeypatch.setenv("SML_GEMM_SPLIT", split)
        moe = sa.MoE(p, 0, 16)
        moe.regime(per256)
        out, sel = sa.DevBuf(T * n_embd * 4), sa.DevBuf(T * k * 4)
        moe.ffn(sa.DevBuf.of(x), T, out, sel)
        outs[split] = (out.read(np.float32).reshape(T, n_embd), sel.read(np.int32).reshape(T, k))
        moe.free()
    got_out, got_sel = outs["1"]
    assert (got_sel[:12] == got_sel[0]).all()
    np.testing.assert_array_equal(outs["0"][0], got_out)
    for t in range(T):
        _, rs, _, ro = oracle_moe(f, x[t], nexp, k, n_embd, per256=per256)
        np.testing.assert_array_equal(got_sel[t], rs, err_msg=f"token {t} routing")
        close(got_out[t], ro, f"moe token {t}")


@pytest.mark.timeout(600)
@pytest.mark.parametrize("per256", [False, True])
def test_moe_mixtral_layer_shape(tmp_path, per256):
    """The Mixtral-shaped layer of the MoE workload at its shape: hidden
    4096, 8 experts of 14336 SwiGLU Q4, router 4096 x 8 ~ N(0, 1/64) (seed
    1005), top-2 with softmax over the chosen, 16 tokens of N(0, 1). Router
    logits, choices and weights equal the oracle's bit for bit (a double sum
    rounded once; the library's restated expf); each token's output within
    1e-3 of the oracle's per-token composition, with the expert inputs
    quantized per 32 (the stepped moe_ffn) or per 256 (moe_ffn_batch): max
    |d| <= 1e-3 max |ref| and rel-RMS <= 1e-3. The expert output is a
    composite -- h is re-quantized to int8 between the products -- and one
    flipped code of h's 14336 moves it by ~1e-4 rel-RMS, so the bound is the
    composite's 1e-3, not a single product's 1e-4."""
    n_embd, n_ff, nexp, k, T = 4096, 14336, 8, 2, 16
    p = tmp_path / "mixtral_layer.ssf"
    sa.synth_model(p, n_layer=1, n_embd=n_embd, n_head=32, n_head_kv=8, n_ff=n_ff, n_vocab=1024, n_expert=nexp,
                   n_expert_used=k, moe_flags=1, rope_theta=1e6, seed=1005)
    f = SSF(p)
    moe = sa.MoE(p, 0, 16)
    moe.regime(per256)
    x = np.random.default_rng(1005).standard_normal((T, n_embd)).astype(np.float32)
    out, sel, w, lg = sa.DevBuf(T * n_embd * 4), sa.DevBuf(T * k * 4), sa.DevBuf(T * k * 4), sa.DevBuf(T * nexp * 4)
    moe.ffn(sa.DevBuf.of(x), T, out, sel, w, lg)
    got_out = out.read(np.float32).reshape(T, n_embd)
    got_sel, got_w = sel.read(np.int32).reshape(T, k), w.read(np.float32).reshape(T, k)
    got_lg = lg.read(np.float32).reshape(T, nexp)
    used = set()
    for t in range(T):
        rl, rs, rw, ro = oracle_moe(f, x[t], nexp, k, n_embd, per256=per256)
        np.testing.assert_array_equal(got_lg[t], rl, err_msg=f"token {t} router logits")
        np.testing.assert_array_equal(got_sel[t], rs, err_msg=f"token {t} routing")
        np.testing.assert_array_equal(got_w[t], rw, err_msg=f"token {t} weights")
        err = np.abs(got_out[t].astype(np.float64) - ro)
        assert err.max() <= 1e-3 * np.abs(ro).max(), (t, err.max())
        assert np.sqrt((err ** 2).mean() / (ro.astype(np.float64) ** 2).mean()) <= 1e-3, t
        used |= set(rs.tolist())
    assert len(used) >= 6, used
    moe.free()


def test_moe_refuses_dense_layer(tmpdir_s):
    p = tmpdir_s / "dense_for_moe.ssf"
    sa.synth_model(p, n_layer=1, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=256, seed=3)
    with pytest.raises(sa.HipError, match="no experts"):
        sa.MoE(p, 0, 4)


def test_tiled_copy_gives_the_same_bits(tmpdir_s):
    # SML_TILED=1 (read once per process): the MFMA GEMM reads each Q4
    # matrix's tiled copy, byte for byte what it loads from the rows, so its
    # outputs equal the untiled run's bit for bit (per-32 and per-256, plain
    # and SwiGLU, persistent and not)
    import subprocess
    import sys as _sys
    code = r'''
import sys, numpy as np
sys.path.insert(0, sys.argv[1])
import sheep_amd as sa
p = sys.argv[2]
rng = np.random.default_rng(77)
out = {}
for rows, cols in ((4096, 4096), (8192, 14336)):
    sa.synth_matrix(p, rows, cols, nbits=4, seed=rows + cols)
    g, u = sa.Mat.from_file(p, "w"), sa.Mat.from_file(p, "w")
    M = 13
    q = sa.DevBuf.of(rng.integers(-127, 128, M * cols).astype(np.int8))
    s32 = (np.abs(rng.standard_normal(M * cols // 32)) * 0.01).astype(np.float32)
    s = sa.DevBuf.of(s32)
    s256 = sa.DevBuf.of(np.repeat(s32.reshape(-1, 8)[:, :1], 8, axis=1).reshape(-1))
    uu = sa.DevBuf.of(rng.integers(-2000, 2000, M * cols // 32).astype(np.int32))
    y = sa.DevBuf(M * rows * 4)
    for sb, sc in ((False, s), (True, s256)):
        sa.gemm(g, q, sc, uu, M, y, per256=sb)
        out[f"{rows}_{sb}_plain"] = y.read(np.float32)
        sa.gemm_swiglu(g, u, q, sc, uu, M, y, per256=sb)
        out[f"{rows}_{sb}_swiglu"] = y.read(np.float32)
np.savez(sys.argv[3], **out)
'''
    import os
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = {}
    for t in ("0", "1"):
        f = str(tmpdir_s / f"tiled_{t}.npz")
        r = subprocess.run([_sys.executable, "-c", code, root, str(tmpdir_s / f"tm_{t}.ssf"), f],
                           env=dict(os.environ, SML_TILED=t), capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stderr[-2000:]
        res[t] = np.load(f)
    for k in res["0"].files:
        assert np.array_equal(res["0"][k], res["1"][k]), k


# (moe_flags, moe_scale, groups, topk_group, exp_bias, shared expert width, its gate)
MOE_MODES = {
    "v3_sigmoid_bias_groups_shared": (3, 2.5, 4, 2, True, 1024, True),
    "sigmoid_bias": (2, 0.0, 1, 1, True, 0, False),
    "softmax_groups_best_one": (9, 1.0, 4, 1, False, 0, False),
    "greedy_scaled_shared_ungated": (0, 1.5, 1, 1, False, 768, False),
    "sparsemixer": (4, 0.01, 1, 1, False, 0, False),
    "mixtral_shared_gated": (1, 0.0, 1, 1, False, 1024, True),
}


@pytest.mark.parametrize("name", list(MOE_MODES))
def test_moe_routing_modes(tmpdir_s, name):
    """Every routing mode of sml_moe_route (sigmoid or softmax scores, the
    correction bias, grouped choice by a group's best one or two, the weight
    scale, PhiMoE's sparsemixer) and a shared expert with or without its
    sigmoid gate, on one MoE layer of 16 experts (top 4) for 16 tokens: the
    choices and weights equal the oracle's restatement (itself equal to the
    reference's sml_moe_route bit for bit) fed the GPU's own logits, and each
    token's output is within 1e-3 of the oracle's composition, the shared
    expert's gated output added after the routed ones."""
    flags, scale, groups, tg, bias, shff, shgate = MOE_MODES[name]
    n_embd, n_ff, nexp, k, T = 1024, 512, 16, 4, 16
    p = tmpdir_s / f"moe_mode_{name}.ssf"
    if not p.exists():
        sa.synth_model(p, n_layer=1, n_embd=n_embd, n_head=8, n_head_kv=2, n_ff=n_ff, n_vocab=512, n_expert=nexp,
                       n_expert_used=k, moe_flags=flags, moe_scale=scale, moe_groups=groups, moe_topk_group=tg,
                       exp_bias=bias, n_ff_shexp=shff, shexp_gate=shgate, random_perm=True,
                       router_sigma=0.5, seed=2000 + flags)
    f = SSF(p)
    moe = sa.MoE(p, 0, 16)
    rng = np.random.default_rng(flags + 40)
    x = rng.standard_normal((T, n_embd)).astype(np.float32)
    out, sel, w, lg = sa.DevBuf(T * n_embd * 4), sa.DevBuf(T * k * 4), sa.DevBuf(T * k * 4), sa.DevBuf(T * nexp * 4)
    xd = sa.DevBuf.of(x)
    print(f"moe mode {name}", flush=True)
    moe.ffn(xd, T, out, sel, w, lg)
    got_out = out.read(np.float32).reshape(T, n_embd)
    got_sel = sel.read(np.int32).reshape(T, k)
    got_w = w.read(np.float32).reshape(T, k)
    got_lg = lg.read(np.float32).reshape(T, nexp)
    eb = np.ascontiguousarray(f["blk.0.exp_probs_b.weight"].f32) if bias else None
    router = np.ascontiguousarray(f["blk.0.ffn_gate_inp.weight"].f32)
    distinct = set()
    for t in range(T):
        rl = np.zeros(nexp, np.float32)
        ob.oracle().orc_router(router.ctypes.data, x[t].ctypes.data, nexp, n_embd, rl.ctypes.data)
        np.testing.assert_allclose(got_lg[t], rl, rtol=1e-6, atol=1e-6)
        rs, rw = np.zeros(k, np.int32), np.zeros(k, np.float32)
        lt = np.ascontiguousarray(got_lg[t])
        ob.oracle().orc_moe_route2(lt.ctypes.data, nexp, k, flags, scale, groups, tg,
                                   eb.ctypes.data if bias else None, rs.ctypes.data, rw.ctypes.data)
        np.testing.assert_array_equal(got_sel[t], rs, err_msg=f"{name} token {t} choices")
        np.testing.assert_array_equal(got_w[t].view(np.uint32), rw.view(np.uint32), err_msg=f"{name} token {t} weights")
        distinct.update(rs.tolist())
        acc = np.zeros(n_embd, np.float32)
        for j in range(k):
            g, u, d = (f[f"blk.0.ffn_{kind}.{int(rs[j])}.weight"] for kind in ("gate", "up", "down"))
            qa = ob.quantize_act(np.ascontiguousarray(x[t][g.perm]))
            yg, yu = ob.matvec(g, *qa), ob.matvec(u, *qa)
            ob.oracle().orc_silu_mul(yg.ctypes.data, yu.ctypes.data, len(yg))
            acc += rw[j] * ob.matvec(d, *ob.quantize_act(np.ascontiguousarray(yg[d.perm])))
        if shff:
            g, u, d = (f[f"blk.0.ffn_{kind}_shexp.weight"] for kind in ("gate", "up", "down"))
            qa = ob.quantize_act(np.ascontiguousarray(x[t][g.perm]))
            yg, yu = ob.matvec(g, *qa), ob.matvec(u, *qa)
            ob.oracle().orc_silu_mul(yg.ctypes.data, yu.ctypes.data, len(yg))
            ysh = ob.matvec(d, *ob.quantize_act(np.ascontiguousarray(yg[d.perm])))
            sg = 1.0
            if shgate:
                gv = f["blk.0.ffn_gate_inp_shexp.weight"].f32.astype(np.float64)
                sg = np.float32(1.0) / (np.float32(1.0) + np.float32(np.exp(-np.float64(np.float32(gv @ x[t].astype(np.float64))))))
            acc += np.float32(sg) * ysh
        close(got_out[t], acc, f"{name} token {t}")
    assert len(distinct) >= 6, (name, distinct)          # the tokens reach many experts
