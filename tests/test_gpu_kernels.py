"""GPU parity of each kernel against the oracle on the same seeded inputs.

Integer work (unpacked codes, int8 activation codes/scales/sums, argmax) is
bit-exact. Float outputs (GEMV, attention) must agree within 1e-3 relative:
    max|gpu - oracle| <= 1e-3 * max|oracle|   and   rel-RMS <= 1e-4.
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


def dev_quantize(x, perm=None, per256=False, w=None, eps=1e-6):
    xd = sa.DevBuf.of(np.ascontiguousarray(x, np.float32))
    act = sa.Act(len(x))
    pd = sa.DevBuf.of(np.ascontiguousarray(perm, np.int32)) if perm is not None else None
    wd = sa.DevBuf.of(np.ascontiguousarray(w, np.float32)) if w is not None else None
    sa.normq(xd, act, perm=pd, w=wd, eps=eps, per256=per256)
    return act


# ------------------------------------------------------------ activations

@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("per256", [False, True])
def test_quantize_bitexact(seed, per256):
    rng = np.random.default_rng(seed)
    n = 14336
    x = (rng.standard_normal(n) * 10.0 ** rng.uniform(-3, 3)).astype(np.float32)
    x[:32] = 0.0
    x[32:64] = np.arange(32, dtype=np.float32) * 0.5
    perm = rng.permutation(n).astype(np.int32) if seed % 2 else None
    act = dev_quantize(x, perm=perm, per256=per256)
    xg = x[perm] if perm is not None else x
    want = ob.quantize_act(xg, per256=per256)
    for got, exp, name in zip(act.read(), want, ("q", "scale", "sums")):
        np.testing.assert_array_equal(got, exp, err_msg=name)


def test_quantize_golden():
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "act_quant.npz"))
    for i in range(2):
        for per256 in (0, 1):
            got = dev_quantize(g[f"x{i}"], per256=bool(per256)).read()
            for a, b in zip(got, (g[f"q{i}_{per256}"], g[f"s{i}_{per256}"], g[f"u{i}_{per256}"])):
                np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("n", [1536, 4096])
def test_normq_bitexact(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
    perm = rng.permutation(n).astype(np.int32)
    act = dev_quantize(x, perm=perm, w=w, eps=1e-6)
    normed = np.zeros(n, np.float32)
    ob.oracle().orc_rms_norm(normed.ctypes.data, x.ctypes.data, w.ctypes.data, n, 1e-6)
    for a, b in zip(act.read(), ob.quantize_act(normed[perm])):
        np.testing.assert_array_equal(a, b)


# ------------------------------------------------------------ unpack

@pytest.mark.parametrize("nb", range(2, 9))
def test_unpack_bitexact(tmpdir_s, nb):
    p = tmpdir_s / f"u{nb}.ssf"
    sa.synth_matrix(p, 96, 1536, nbits=nb, random_perm=True, seed=300 + nb)
    t = SSF(p)["w"]
    m = sa.Mat.from_file(p, "w")
    got = sa.unpack(m, 0, 96)
    want = np.stack([ob.unpack(t, r) for r in range(96)])
    np.testing.assert_array_equal(got, want)


# ------------------------------------------------------------ GEMV

def gemv_case(tmpdir_s, rows, cols, nb, perm=False, seed=1, check_ref=False):
    p = tmpdir_s / f"g_{rows}x{cols}_q{nb}_{int(perm)}_{seed}.ssf"
    if not p.exists():
        sa.synth_matrix(p, rows, cols, nbits=nb, random_perm=perm, seed=seed)
    f = SSF(p)
    t = f["w"]
    x = np.random.default_rng(seed).standard_normal(cols).astype(np.float32)
    m = sa.Mat.from_file(p, "w")
    act = dev_quantize(x, perm=t.perm)
    y = sa.DevBuf(rows * 4)
    sa.matvec(m, act, y)
    got = y.read(np.float32)
    q, s, u = ob.quantize_act(x[t.perm])
    close(got, ob.matvec(t, q, s, u), f"{rows}x{cols} Q{nb}")
    if check_ref and ob.have_ref():
        close(got, ob.ref_matvec(t, q, s, u), f"{rows}x{cols} Q{nb} vs reference build")
    return got


@pytest.mark.parametrize("nb", range(2, 9))
def test_gemv_small(tmpdir_s, nb):
    gemv_case(tmpdir_s, 256, 1536, nb, perm=True, seed=10 + nb, check_ref=True)


@pytest.mark.parametrize("perm", [False, True])
def test_gemv_single_q4_8960x1536(tmpdir_s, perm):
    """The single-GEMV workload: Qwen2.5-1.5B FFN-up shape, rows 8960 x cols 1536."""
    gemv_case(tmpdir_s, 8960, 1536, 4, perm=perm, seed=1001, check_ref=True)


@pytest.mark.parametrize("shape", [(4096, 14336), (14336, 4096)])
@pytest.mark.parametrize("nb", [2, 3, 4, 5, 6, 8])
def test_gemv_width_sweep(tmpdir_s, shape, nb):
    gemv_case(tmpdir_s, shape[0], shape[1], nb, seed=1004)


def test_gemv_rows_not_multiple_of_block(tmpdir_s):
    gemv_case(tmpdir_s, 257, 512, 4, seed=3)
    gemv_case(tmpdir_s, 1, 128, 4, seed=4)


def test_gemv_repeat_is_deterministic(tmpdir_s):
    a = gemv_case(tmpdir_s, 4096, 4096, 4, seed=5)
    b = gemv_case(tmpdir_s, 4096, 4096, 4, seed=5)
    np.testing.assert_array_equal(a, b)


def test_swiglu(tmpdir_s):
    p = tmpdir_s / "ffn.ssf"
    sa.synth_model(p, n_layer=1, n_embd=1536, n_head=12, n_head_kv=2, n_ff=8960, n_vocab=256, seed=77)
    f = SSF(p)
    g, u = f["blk.0.ffn_gate.weight"], f["blk.0.ffn_up.weight"]
    x = np.random.default_rng(0).standard_normal(1536).astype(np.float32)
    act = dev_quantize(x, perm=g.perm)
    mg, mu = sa.Mat.from_file(p, g.name), sa.Mat.from_file(p, u.name)
    h = sa.DevBuf(8960 * 4)
    sa.matvec_swiglu(mg, mu, act, h)
    q, s, su = ob.quantize_act(x[g.perm])
    yg, yu = ob.matvec(g, q, s, su), ob.matvec(u, q, s, su)
    ob.oracle().orc_silu_mul(yg.ctypes.data, yu.ctypes.data, 8960)
    close(h.read(np.float32), yg, "swiglu")


# ------------------------------------------------------------ fused activation prologue, h quantization

@pytest.mark.parametrize("nb", [4, 3, 6, 8])
@pytest.mark.parametrize("cols,use_perm,use_norm", [(1536, True, True), (4096, False, True), (4096, True, False),
                                                     (2048, False, False)])
def test_matvec_normq_equals_normq_then_matvec(tmpdir_s, nb, cols, use_perm, use_norm):
    """The prologue computes the normq kernel's activation bit for bit, so the
    fused GEMV's output equals normq + matvec exactly; both match the oracle."""
    p = tmpdir_s / f"fz{nb}_{cols}_{int(use_perm)}.ssf"
    if not p.exists():
        sa.synth_matrix(p, 1000, cols, nbits=nb, random_perm=use_perm, seed=900 + nb + cols)
    t = SSF(p)["w"]
    m = sa.Mat.from_file(p, "w")
    rng = np.random.default_rng(cols + nb)
    x = (rng.standard_normal(cols) * 3).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
    perm = t.perm.astype(np.int32) if use_perm else None
    act = dev_quantize(x, perm=perm, w=w if use_norm else None, eps=1e-5)
    y0, y1 = sa.DevBuf(1000 * 4), sa.DevBuf(1000 * 4)
    sa.matvec(m, act, y0)
    xd, wd = sa.DevBuf.of(x), sa.DevBuf.of(w)
    pd = sa.DevBuf.of(perm) if use_perm else None
    sa.matvec_normq(m, xd, y1, w=wd if use_norm else None, perm=pd, eps=1e-5)
    got = y1.read(np.float32)
    np.testing.assert_array_equal(got, y0.read(np.float32))
    v = x
    if use_norm:
        v = np.zeros(cols, np.float32)
        ob.oracle().orc_rms_norm(v.ctypes.data, x.ctypes.data, w.ctypes.data, cols, np.float32(1e-5))
    q, sc, su = ob.quantize_act(v[perm] if use_perm else v)
    close(got, ob.matvec(t, q, sc, su), "matvec_normq")


@pytest.mark.parametrize("n_embd,nb,xin,perm", [(1536, 4, True, True), (1536, 5, False, False),
                                                (4096, 4, True, False), (4096, 8, True, True)])
def test_swiglu_h_quantization(tmpdir_s, n_embd, nb, xin, perm):
    """The h-quantizing SwiGLU kernel (16 lanes per row) agrees with the plain
    SwiGLU to float rounding of the same sums, and its per-32 quantization of
    its own h equals the normq kernel's (no norm, in order) bit for bit."""
    p = tmpdir_s / f"ffnh{n_embd}_{nb}_{int(perm)}.ssf"
    n_ff = 2048 + 128       # 68 groups of h: 68 workgroups of the h kernel
    if not p.exists():
        sa.synth_model(p, n_layer=1, n_embd=n_embd, n_head=n_embd // 128, n_head_kv=2, n_ff=n_ff, n_vocab=256, nbits=nb,
                       random_perm=perm, seed=78 + nb)
    f = SSF(p)
    g, u = f["blk.0.ffn_gate.weight"], f["blk.0.ffn_up.weight"]
    rng = np.random.default_rng(n_embd)
    x = (rng.standard_normal(n_embd) * 2).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(n_embd)).astype(np.float32)
    gp = g.perm.astype(np.int32) if g.perm is not None else None
    act = dev_quantize(x, perm=gp, w=w, eps=1e-5)
    mg, mu = sa.Mat.from_file(p, g.name), sa.Mat.from_file(p, u.name)
    h0, h1 = sa.DevBuf(n_ff * 4), sa.DevBuf(n_ff * 4)
    sa.matvec_swiglu(mg, mu, act, h0)
    hact = sa.Act(n_ff)
    if xin:
        sa.matvec_swiglu_fused(mg, mu, h1, x=sa.DevBuf.of(x), w=sa.DevBuf.of(w), eps=1e-5,
                               perm=sa.DevBuf.of(gp) if gp is not None else None, hact=hact)
    else:
        sa.matvec_swiglu_fused(mg, mu, h1, act=act, hact=hact)
    h = h1.read(np.float32)
    h_ref = h0.read(np.float32)
    assert np.abs(h - h_ref).max() <= 1e-6 * np.abs(h_ref).max()
    for a, b, name in zip(hact.read(), ob.quantize_act(h), ("q", "scale", "sums")):
        np.testing.assert_array_equal(a, b, err_msg=name)


# ------------------------------------------------------------ embed, attention, argmax

@pytest.mark.parametrize("nb", [2, 3, 4, 5, 6, 7, 8])
def test_embed(tmpdir_s, nb):
    p = tmpdir_s / f"emb{nb}.ssf"
    sa.synth_matrix(p, 1000, 1536, nbits=nb, random_perm=True, seed=500 + nb)
    t = SSF(p)["w"]
    m = sa.Mat.from_file(p, "w")
    for tok in (0, 537, 999):
        td = sa.DevBuf.of(np.array([tok], np.int32))
        pd = sa.DevBuf.of(t.perm.astype(np.int32))
        x = sa.DevBuf(1536 * 4)
        assert sa.lib().sml_hip_embed(m.h, td.ptr, pd.ptr, x.ptr) == 0
        want = np.zeros(1536, np.float32)
        want[t.perm] = ob.dequant_row(t, tok)
        np.testing.assert_array_equal(x.read(np.float32), want)
        # in storage order (no permutation: Q4 takes the vector path)
        assert sa.lib().sml_hip_embed(m.h, td.ptr, None, x.ptr) == 0
        np.testing.assert_array_equal(x.read(np.float32), ob.dequant_row(t, tok))


@pytest.mark.parametrize("heads", [(12, 2), (32, 8)])
def test_attention(heads):
    H, KV = heads
    hd, n_ctx, half = 128, 512, 64
    rng = np.random.default_rng(H)
    cos_t = np.zeros(n_ctx * half, np.float32)
    sin_t = np.zeros(n_ctx * half, np.float32)
    ob.oracle().orc_rope_table(1e6, half, n_ctx, cos_t.ctypes.data, sin_t.ctypes.data)
    kvd = KV * hd
    kc = np.zeros((n_ctx, kvd), np.uint16)
    vc = np.zeros((n_ctx, kvd), np.uint16)
    dkc, dvc = sa.DevBuf.of(kc), sa.DevBuf.of(vc)
    dcos, dsin = sa.DevBuf.of(cos_t), sa.DevBuf.of(sin_t)
    part = sa.DevBuf(sa.lib().sml_hip_attn_part_floats(H, hd, n_ctx) * 4)
    out = sa.DevBuf(H * hd * 4)
    scratch = np.zeros(n_ctx, np.float32)
    for pos in range(0, 300):
        q = rng.standard_normal(H * hd).astype(np.float32)
        k = rng.standard_normal(kvd).astype(np.float32)
        v = rng.standard_normal(kvd).astype(np.float32)
        dq, dk, dv = sa.DevBuf.of(q), sa.DevBuf.of(k), sa.DevBuf.of(v)
        dpos = sa.DevBuf.of(np.array([pos], np.int32))
        rc = sa.lib().sml_hip_attention(dq.ptr, dk.ptr, dv.ptr, dkc.ptr, dvc.ptr, dcos.ptr, dsin.ptr, dpos.ptr,
                                        H, KV, hd, n_ctx, part.ptr, out.ptr)
        assert rc == 0, sa.lib().sml_hip_last_error()
        # oracle: rotate, store fp16, attend
        qr, kr = q.copy(), k.copy()
        ob.oracle().orc_rope(qr.ctypes.data, H, hd, half, cos_t[pos * half:].ctypes.data, sin_t[pos * half:].ctypes.data)
        ob.oracle().orc_rope(kr.ctypes.data, KV, hd, half, cos_t[pos * half:].ctypes.data, sin_t[pos * half:].ctypes.data)
        kc[pos] = kr.astype(np.float16).view(np.uint16)
        vc[pos] = v.astype(np.float16).view(np.uint16)
        if pos not in (0, 1, 63, 64, 65, 127, 200, 299):
            continue
        np.testing.assert_array_equal(dkc.read(np.uint16).reshape(n_ctx, kvd)[pos], kc[pos])
        np.testing.assert_array_equal(dvc.read(np.uint16).reshape(n_ctx, kvd)[pos], vc[pos])
        want = np.zeros(H * hd, np.float32)
        inv = np.float32(1) / np.sqrt(np.float32(hd))
        for h in range(H):
            kh = h // (H // KV)
            ob.oracle().orc_attn_head(qr[h * hd:].ctypes.data, kc[:, kh * hd:].ctypes.data, vc[:, kh * hd:].ctypes.data,
                                      kvd, pos, hd, inv, scratch.ctypes.data, want[h * hd:].ctypes.data)
        close(out.read(np.float32), want, f"attention pos {pos}")


def test_argmax_first_max():
    """One workgroup below 8192 logits, two stages (per-workgroup pairs, then
    one workgroup) from there: ties across workgroups, ragged tails, NaN and
    all -inf keep the reference loop's answer."""
    rng = np.random.default_rng(0)
    cases = [(151936, "tie"), (128256, None), (1000, "tie"), (5, None), (8191, "tie"), (8192, "tie"),
             (8193, "tie"), (151937, "tie"), (128256, "nan"), (128256, "nan0"), (9000, "-inf"),
             (5_000_003, "tie")]
    for n, kind in cases:
        lg = rng.standard_normal(n).astype(np.float32)
        if kind == "tie":
            lg[n // 3] = lg[n - 1] = lg.max() + 1.0
        elif kind == "nan":
            lg[n // 2] = np.nan
            lg[n // 5] = lg[n - 2] = np.nanmax(lg) + 1.0
        elif kind == "nan0":
            lg[0] = np.nan
        elif kind == "-inf":
            lg[:] = -np.inf
        d = sa.DevBuf.of(lg)
        t = sa.DevBuf(4)
        assert sa.lib().sml_hip_argmax(d.ptr, n, t.ptr) == 0
        assert int(t.read(np.int32)[0]) == ob.oracle().orc_argmax(lg.ctypes.data, n), (n, kind)


def test_copy_calibration_kernel():
    """The counter-calibration copy moves exactly the bytes asked for."""
    rng = np.random.default_rng(5)
    for n in (16, 4096 + 48, 3 << 20):
        src = rng.integers(0, 256, n + 64, dtype=np.uint8)
        s, d = sa.DevBuf.of(src), sa.DevBuf.of(np.zeros(n + 64, np.uint8))
        assert sa.lib().sml_hip_copy(d.ptr, s.ptr, n) == 0
        out = d.read(np.uint8)
        assert np.array_equal(out[:n], src[:n]) and not out[n:].any()
    assert sa.lib().sml_hip_copy(d.ptr, s.ptr, 17) == -1


# ------------------------------------------------------------ GPTQ-style 4-bit

@pytest.mark.parametrize("rows,cols", [(256, 1024), (1000, 1152), (4096, 14336), (14336, 4096)])
def test_gptq_gemv(rows, cols):
    from sheep_amd import gptq as gq
    qw, qz, sc = gq.synth(rows, cols, seed=rows + cols)
    m = gq.GptqMat(qw, qz, sc, rows, cols)
    x = np.random.default_rng(cols).standard_normal(cols).astype(np.float32)
    y = sa.DevBuf(rows * 4)
    m.matvec(sa.DevBuf.of(x), y)
    close(y.read(np.float32), ob.gptq_matvec(qw, qz, sc, rows, cols, x), f"gptq {rows}x{cols}")


@pytest.mark.parametrize("rows,cols", [(1000, 1152), (4096, 14336), (14336, 4096)])
def test_gptq_folded_reduce_equals_reduce_launch(rows, cols, monkeypatch):
    """The split-K sum done by each output block's last workgroup (counters
    cleared by that workgroup) equals the separate sml_gptq_reduce launch bit
    for bit, at 2 and 4 outputs per lane, over several calls in a row on
    different inputs (so every counter was left at zero)."""
    from sheep_amd import gptq as gq
    qw, qz, sc = gq.synth(rows, cols, seed=rows + 2 * cols)
    m = gq.GptqMat(qw, qz, sc, rows, cols)
    rng = np.random.default_rng(rows)
    xs = [sa.DevBuf.of(rng.standard_normal(cols).astype(np.float32)) for _ in range(3)]
    y = sa.DevBuf(rows * 4)
    for opl in ("2", "4"):
        monkeypatch.setenv("SML_GPTQ_OPL", opl)
        for i, x in enumerate(xs):
            got = {}
            for fold in ("1", "0", "1"):
                monkeypatch.setenv("SML_GPTQ_FOLD", fold)
                m.matvec(x, y)
                got.setdefault(fold, []).append(y.read(np.float32))
            np.testing.assert_array_equal(got["1"][0], got["0"][0], err_msg=f"opl {opl} call {i}")
            np.testing.assert_array_equal(got["1"][1], got["0"][0], err_msg=f"opl {opl} call {i} again")


@pytest.mark.parametrize("rows,cols,zero_add", [(4096, 14336, 1), (1000, 1152, 0)])
def test_gptq_unpack_bitexact(rows, cols, zero_add):
    from sheep_amd import gptq as gq
    qw, qz, sc = gq.synth(rows, cols, seed=7 + rows)
    rng = np.random.default_rng(rows)
    qz = rng.integers(0, 1 << 32, qz.shape, dtype=np.uint64).astype(np.uint32).view(np.int32)
    m = gq.GptqMat(qw, qz, sc, rows, cols, zero_add=zero_add)
    for r0, n in ((0, 8), (rows - 5, 5), (rows // 2, 3)):
        c, z = m.unpack(r0, n)
        for i in range(n):
            wc, wz = ob.gptq_unpack_row(qw, qz, rows, cols, r0 + i, zero_add=zero_add)
            np.testing.assert_array_equal(c[i], wc)
            np.testing.assert_array_equal(z[i], wz)


@pytest.mark.parametrize("rows,cols", [(4096, 14336), (1000, 1152)])
def test_gptq_desc_act(rows, cols):
    """A desc_act matrix (g_idx scattering each group's 128 inputs over the
    row): the upload reorders the input columns stably by g_idx and the GEMV
    gathers x the same way. Codes and zeros come back in that order, bit for
    bit the file's codes of inputs argsort(g_idx, stable); the GEMV within 1e-3
    of the oracle's g_idx dequantize-then-dot; an identity g_idx gives the
    plain upload's output bit for bit."""
    from sheep_amd import gptq as gq
    qw, qz, sc = gq.synth(rows, cols, seed=rows + 3)
    rng = np.random.default_rng(cols + 5)
    qz = rng.integers(0, 1 << 32, qz.shape, dtype=np.uint64).astype(np.uint32).view(np.int32)
    g_idx = gq.desc_act_gidx(cols, rows)
    order = np.argsort(g_idx, kind="stable")
    m = gq.GptqMat(qw, qz, sc, rows, cols, g_idx=g_idx)
    for r0, n in ((0, 8), (rows - 5, 5)):
        c, z = m.unpack(r0, n)
        for i in range(n):
            wc, wz = ob.gptq_unpack_row(qw, qz, rows, cols, r0 + i)
            np.testing.assert_array_equal(c[i], wc[order])
            np.testing.assert_array_equal(z[i], wz)
    x = rng.standard_normal(cols).astype(np.float32)
    xd = sa.DevBuf.of(x)
    y = sa.DevBuf(rows * 4)
    m.matvec(xd, y)
    close(y.read(np.float32), ob.gptq_matvec_gidx(qw, qz, sc, g_idx, rows, cols, x), f"gptq desc_act {rows}x{cols}")
    ident = gq.GptqMat(qw, qz, sc, rows, cols, g_idx=(np.arange(cols) // 128).astype(np.int32))
    plain = gq.GptqMat(qw, qz, sc, rows, cols)
    ya, yb = sa.DevBuf(rows * 4), sa.DevBuf(rows * 4)
    ident.matvec(xd, ya)
    plain.matvec(xd, yb)
    np.testing.assert_array_equal(ya.read(np.float32), yb.read(np.float32))
    bad = np.array(g_idx)
    bad[0] = bad[1] if bad[0] != bad[1] else (bad[1] + 1) % (cols // 128)
    with pytest.raises(sa.HipError):
        gq.GptqMat(qw, qz, sc, rows, cols, g_idx=bad)


@pytest.mark.parametrize("rows,cols,with_zeros", [(4096, 14336, True), (1000, 1152, False)])
def test_awq_unpack_and_gemv(rows, cols, with_zeros):
    """The AWQ layout (output-packed words, nibble order 0,4,1,5,2,6,3,7;
    default zero 8 without qzeros), repacked at upload into the GPTQ device
    layout: codes and zeros bit-exact with the oracle's AWQ reading, the
    GEMV within 1e-3 of the oracle's dequantize-then-dot."""
    from sheep_amd import gptq as gq
    rng = np.random.default_rng(rows + cols)
    ngr = cols // 128
    qw = rng.integers(0, 1 << 32, (cols, rows // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
    qz = rng.integers(0, 1 << 32, (ngr, rows // 8), dtype=np.uint64).astype(np.uint32).view(np.int32) \
        if with_zeros else None
    sc = (np.abs(rng.standard_normal((ngr, rows))) * 0.02 / 7).astype(np.float16)
    m = gq.GptqMat(qw, qz, sc, rows, cols, awq=True)
    for r0, n in ((0, 8), (rows - 5, 5), (rows // 2, 3)):
        c, z = m.unpack(r0, n)
        for i in range(n):
            wc, wz = ob.awq_unpack_row(qw, qz, rows, cols, r0 + i)
            np.testing.assert_array_equal(c[i], wc)
            np.testing.assert_array_equal(z[i], wz)
    x = rng.standard_normal(cols).astype(np.float32)
    y = sa.DevBuf(rows * 4)
    m.matvec(sa.DevBuf.of(x), y)
    W = np.stack([ob.awq_dequant_row(qw, qz, sc, rows, cols, r) for r in range(rows)]).astype(np.float64)
    close(y.read(np.float32), (W @ x.astype(np.float64)).astype(np.float32), f"awq {rows}x{cols}")


# ------------------------------------------------------------ loader: declared sizes against the shape

@pytest.mark.parametrize("field", ["n0", "sd_bytes", "sq_bytes", "md_bytes", "mq_bytes", "p0"])
def test_short_record_is_refused(tmp_path, field):
    """A record whose declared array sizes pass the file-range checks but are
    shorter than its shape reads (or whose plane offset is 0) is refused at
    upload with a reason, and sml_gpu_open returns 0 instead of reading past
    the mapping."""
    import re
    import shutil
    import struct
    from sheep_amd.ssf import REC_FIELDS, REC_FMT, REC_SIZE
    codes = []
    for n, c in re.findall(r"(\d*)([a-zA-Z])", REC_FMT[1:]):
        codes += [n + c] if c == "s" else [c] * (int(n) if n else 1)
    off = struct.calcsize("<" + "".join(codes[:REC_FIELDS.index(field)]))
    src = tmp_path / "base.ssf"
    sa.synth_model(src, n_layer=1, n_embd=256, n_head=2, n_head_kv=1, n_ff=512, n_vocab=300, seed=3)
    f = SSF(src)
    name = "blk.0.ffn_down.weight"
    i = list(f.tensors).index(name)
    p = tmp_path / f"short_{field}.ssf"
    shutil.copy(src, p)
    with open(p, "r+b") as fh:
        fh.seek(f.hdr["table_off"] + i * REC_SIZE + off)
        fh.write(struct.pack("<Q", 0 if field == "p0" else f[name].rec[field] // 2))
        if field == "p0":       # no plane at all: offset and size 0 pass the file-range checks
            fh.seek(f.hdr["table_off"] + i * REC_SIZE + struct.calcsize("<" + "".join(codes[:REC_FIELDS.index("n0")])))
            fh.write(struct.pack("<Q", 0))
    assert not sa.lib().sml_hip_mat_from_file(str(p).encode(), name.encode())
    err = sa.lib().sml_hip_last_error()
    assert b"shorter" in err or b"missing" in err, err
    why = sa.ctypes.create_string_buffer(512)
    assert sa.lib().sml_gpu_open(str(p).encode(), 64, 1, 0, why, 512) == 0
    assert why.value
