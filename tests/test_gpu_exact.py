"""Exact mode on the GPU: the reference CPU path's float order, bit for bit.

With exact mode on (sml_hip_set_exact for single launches, SML_EXACT=1 at
sml_gpu_open for the forward pass), the Q4/Q8 GEMVs run the reference
build's eight superblock lanes with its fused products and its lane fold
(sml/sml-kernel.c:572-727,836-866), norms sum their squares as its serial
double chain, and attention runs its score lanes, serial softmax sum and
serial P.V chains with the C library's expf (sml/sml-run.c:147-152,180-287).
Every output is compared bit for bit: with the oracle (itself bit-exact with
the reference build on the CPU) and, where it is built, with the reference's
own kernels and its sml_forward.
"""
import contextlib
import os

import numpy as np
import pytest

import sheep_amd as sa
from oracle import bind as ob
from sheep_amd.ssf import SSF

pytestmark = pytest.mark.gpu
needs_ref = pytest.mark.skipif(not ob.have_ref(), reason="oracle/_ref (the reference's CPU engine) is not built")


@pytest.fixture(scope="module", autouse=True)
def device():
    sa.init(0)


@contextlib.contextmanager
def exact_mode():
    sa.lib().sml_hip_set_exact(1)
    try:
        yield
    finally:
        sa.lib().sml_hip_set_exact(0)


def same_bits(got, want, what):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, (f"{what}: {bad.size} of {got.size} differ, first at {bad[0]}: "
                           f"{got[bad[0]]!r} vs {want[bad[0]]!r}")


def dev_act(x, perm=None, w=None, eps=1e-6):
    act = sa.Act(len(x))
    sa.normq(sa.DevBuf.of(np.ascontiguousarray(x, np.float32)), act,
             perm=sa.DevBuf.of(np.ascontiguousarray(perm, np.int32)) if perm is not None else None,
             w=sa.DevBuf.of(np.ascontiguousarray(w, np.float32)) if w is not None else None, eps=eps)
    return act


# ------------------------------------------------------------ kernels

@pytest.mark.parametrize("nb", [4, 8])
@pytest.mark.parametrize("rows,cols", [(8960, 1536), (4096, 14336), (14336, 4096), (300, 384), (64, 128)])
def test_exact_gemv_bit_exact(tmpdir_s, nb, rows, cols):
    """Every row equals the oracle's and the reference build's own
    sml_matvec_rows_flat4 / _flat8 bit for bit, including the rows whose
    width ends in half a superblock (384, 128 columns: the four trailing
    lanes the reference adds last)."""
    p = tmpdir_s / f"x_{rows}x{cols}_q{nb}.ssf"
    if not p.exists():
        sa.synth_matrix(p, rows, cols, nbits=nb, random_perm=True, seed=rows + cols + nb)
    t = SSF(p)["w"]
    m = sa.Mat.from_file(p, "w")
    x = np.random.default_rng(cols).standard_normal(cols).astype(np.float32)
    act = dev_act(x, perm=t.perm)
    y = sa.DevBuf(rows * 4)
    with exact_mode():
        sa.matvec(m, act, y)
    got = y.read(np.float32)
    q, s, u = ob.quantize_act(x[t.perm])
    same_bits(got, ob.matvec(t, q, s, u), f"{rows}x{cols} Q{nb} vs oracle")
    if ob.have_ref():
        same_bits(got, ob.ref_matvec(t, q, s, u), f"{rows}x{cols} Q{nb} vs the reference's kernel")


@pytest.mark.parametrize("nb", [4, 8])
@pytest.mark.parametrize("rows,cols,boundary", [(6144, 4096, False), (2048, 1536, False), (384, 4096, True),
                                                 (300, 1536, True)])
def test_exact_gemv_fused_norm_bit_exact(tmpdir_s, nb, rows, cols, boundary):
    """The exact GEMV with its RMSNorm/gather/quantize prologue (the decode
    step's q/k/v form): every row equals the oracle's norm, quantization and
    GEMV in the reference's order, also on inputs whose sum of squares sits
    on a float rounding boundary (the prologue's serial-chain fallback)."""
    import norm_cases as nc
    p = tmpdir_s / f"xn_{rows}x{cols}_q{nb}.ssf"
    if not p.exists():
        sa.synth_matrix(p, rows, cols, nbits=nb, random_perm=True, seed=rows + cols + nb + 7)
    t = SSF(p)["w"]
    m = sa.Mat.from_file(p, "w")
    rng = np.random.default_rng(cols + boundary)
    x = nc.boundary_vector(cols, rng) if boundary else (rng.standard_normal(cols) * 3).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(cols)).astype(np.float32)
    y = sa.DevBuf(rows * 4)
    with exact_mode():
        sa.matvec_normq(m, sa.DevBuf.of(x), y, w=sa.DevBuf.of(w), perm=sa.DevBuf.of(t.perm.astype(np.int32)),
                        eps=1e-5)
    normed = np.zeros(cols, np.float32)
    ob.oracle().orc_rms_norm(normed.ctypes.data, x.ctypes.data, w.ctypes.data, cols, np.float32(1e-5))
    q, s, u = ob.quantize_act(normed[t.perm])
    same_bits(y.read(np.float32), ob.matvec(t, q, s, u), f"{rows}x{cols} Q{nb} fused norm")


@pytest.mark.parametrize("hq", [None, "512", "1024"])
def test_exact_swiglu_fused_norm_bit_exact(tmpdir_s, hq, monkeypatch):
    """The exact SwiGLU GEMV with the prologue (the decode step's gate/up
    form): h equals the oracle's norm, gate, up and SiLU bit for bit; with
    h quantized in the epilogue (32 outputs per workgroup of 512 or 1024
    threads), its codes, scales and sums equal the oracle's quantization
    of that h."""
    if hq:
        monkeypatch.setenv("SML_GEMV_HXWG", hq)
    n_ff = 8960
    p = tmpdir_s / f"xffn{n_ff}.ssf"
    if not p.exists():
        sa.synth_model(p, n_layer=1, n_embd=1536, n_head=12, n_head_kv=2, n_ff=n_ff, n_vocab=256,
                       random_perm=True, seed=n_ff)
    f = SSF(p)
    g, u = f["blk.0.ffn_gate.weight"], f["blk.0.ffn_up.weight"]
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(1536) * 2).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(1536)).astype(np.float32)
    h = sa.DevBuf(n_ff * 4)
    hact = sa.Act(n_ff) if hq else None
    with exact_mode():
        sa.matvec_swiglu_fused(sa.Mat.from_file(p, g.name), sa.Mat.from_file(p, u.name), h, x=sa.DevBuf.of(x),
                               w=sa.DevBuf.of(w), perm=sa.DevBuf.of(g.perm.astype(np.int32)), eps=1e-5,
                               hact=hact)
    normed = np.zeros(1536, np.float32)
    ob.oracle().orc_rms_norm(normed.ctypes.data, x.ctypes.data, w.ctypes.data, 1536, np.float32(1e-5))
    q, s, su = ob.quantize_act(normed[g.perm])
    yg, yu = ob.matvec(g, q, s, su), ob.matvec(u, q, s, su)
    ob.oracle().orc_silu_mul(yg.ctypes.data, yu.ctypes.data, n_ff)
    same_bits(h.read(np.float32), yg, "swiglu with the fused norm")
    if hq:
        for a, b, name in zip(hact.read(), ob.quantize_act(yg), ("q", "scale", "sums")):
            np.testing.assert_array_equal(a, b, err_msg=f"h quantized in the epilogue: {name}")


@pytest.mark.parametrize("n_ff", [8960, 2048 + 128])
def test_exact_swiglu_bit_exact(tmpdir_s, n_ff):
    """gate and up in the reference's order, then its SiLU polynomial
    (sml/sml-run.c:393-426): h equals the oracle's bit for bit."""
    p = tmpdir_s / f"xffn{n_ff}.ssf"
    if not p.exists():
        sa.synth_model(p, n_layer=1, n_embd=1536, n_head=12, n_head_kv=2, n_ff=n_ff, n_vocab=256,
                       random_perm=True, seed=n_ff)
    f = SSF(p)
    g, u = f["blk.0.ffn_gate.weight"], f["blk.0.ffn_up.weight"]
    x = (np.random.default_rng(1).standard_normal(1536) * 2).astype(np.float32)
    act = dev_act(x, perm=g.perm)
    h = sa.DevBuf(n_ff * 4)
    with exact_mode():
        sa.matvec_swiglu(sa.Mat.from_file(p, g.name), sa.Mat.from_file(p, u.name), act, h)
    q, s, su = ob.quantize_act(x[g.perm])
    yg, yu = ob.matvec(g, q, s, su), ob.matvec(u, q, s, su)
    ob.oracle().orc_silu_mul(yg.ctypes.data, yu.ctypes.data, n_ff)
    same_bits(h.read(np.float32), yg, "swiglu")


@pytest.mark.parametrize("n", [1536, 4096, 14336])
def test_exact_normq_bit_exact(n):
    """RMSNorm with the serial double sum, gathered and quantized: codes,
    scales and sums equal the oracle's."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 3).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
    perm = rng.permutation(n).astype(np.int32)
    with exact_mode():
        act = dev_act(x, perm=perm, w=w, eps=1e-5)
    normed = np.zeros(n, np.float32)
    ob.oracle().orc_rms_norm(normed.ctypes.data, x.ctypes.data, w.ctypes.data, n, np.float32(1e-5))
    for a, b, name in zip(act.read(), ob.quantize_act(normed[perm]), ("q", "scale", "sums")):
        np.testing.assert_array_equal(a, b, err_msg=name)


@pytest.mark.parametrize("n", [1536, 4096, 14336])
@pytest.mark.parametrize("with_resid", [False, True])
def test_exact_normq_at_rounding_boundary(n, with_resid):
    """Inputs whose serial sum of squares ends on a float midpoint of ss/n
    while any tree order ends above it (tests/norm_cases.py): the parallel
    sum must fall back to the serial chain, or the norm's scale is one place
    off. Both kernels: the multi-workgroup one, and (with a residual of
    zeros) the one-workgroup one."""
    import norm_cases as nc
    rng = np.random.default_rng(n + with_resid)
    x = nc.boundary_vector(n, rng)
    w = (1 + 0.02 * rng.standard_normal(n)).astype(np.float32)
    perm = rng.permutation(n).astype(np.int32)
    act = sa.Act(n)
    with exact_mode():
        sa.normq(sa.DevBuf.of(x), act, perm=sa.DevBuf.of(perm), w=sa.DevBuf.of(w), eps=1e-5,
                 resid=sa.DevBuf.of(np.zeros(n, np.float32)) if with_resid else None)
    normed = np.zeros(n, np.float32)
    ob.oracle().orc_rms_norm(normed.ctypes.data, x.ctypes.data, w.ctypes.data, n, np.float32(1e-5))
    for a, b, name in zip(act.read(), ob.quantize_act(normed[perm]), ("q", "scale", "sums")):
        np.testing.assert_array_equal(a, b, err_msg=name)


def _serial_sum(x):
    s = np.float32(0)
    for v in np.asarray(x, np.float32):
        s = np.float32(s + v)
    return s


def _sum_cases(rng):
    """Softmax-like values at many lengths, and values built to hit the
    segmented sum's slow paths: exact half-way ties against the running
    sum's last place, zeros, tiny values, a value that crosses several
    binades at once, and lengths that are not whole segments."""
    for n in (1, 2, 63, 64, 65, 1000, 4096, 4097, 16384):
        sc = rng.standard_normal(n) * rng.uniform(0.5, 6)
        e = np.exp((sc - sc.max()).astype(np.float32)).astype(np.float32)
        yield f"softmax {n}", e
    e = np.exp(-rng.random(4096).astype(np.float32) * 4).astype(np.float32)
    # the running sum ends near 1000 (last place 2^-14 there, finer before):
    # values on grids of 2^-15 .. 2^-17 fall half-way between its floats
    for g in (15, 16, 17):
        yield f"ties (multiples of 2^-{g})", (np.round(e * 2 ** g) / 2 ** g).astype(np.float32)
    z = e.copy()
    z[rng.integers(0, 4096, 300)] = 0.0
    z[:100] = np.float32(1e-30)
    yield "zeros and tiny leading values", z
    c = np.full(4096, np.float32(2.0 ** -20))
    c[2000] = np.float32(1.0)
    yield "one value over many binades", c
    yield "all equal", np.full(3000, np.float32(0.3))


def test_softmax_sum_is_the_serial_chain():
    """The exact attention's softmax sum (a serial float chain in the
    reference) computed in segments: bit for bit the chain's result."""
    rng = np.random.default_rng(5)
    out = sa.DevBuf(4)
    for name, e in _sum_cases(rng):
        print(f"softmax sum: {name}", flush=True)
        de = sa.DevBuf.of(e)
        assert sa.lib().sml_hip_softmax_sum(de.ptr, len(e), out.ptr) == 0
        got = out.read(np.float32)[0]
        want = _serial_sum(e)
        assert got.view(np.uint32) == want.view(np.uint32), f"{name}: {got!r} vs {want!r}"


def attention_case(H, KV, n_ctx, positions, exact, seed, hd=128):
    """Fill a cache with random fp16 rows, then run attention at each of
    `positions` (rotating q and k, writing the position's rows) and compare
    the output with the oracle's reference-order attention."""
    half = hd // 2
    rng = np.random.default_rng(seed)
    cos_t = np.zeros(n_ctx * half, np.float32)
    sin_t = np.zeros(n_ctx * half, np.float32)
    ob.oracle().orc_rope_table(5e5, half, n_ctx, cos_t.ctypes.data, sin_t.ctypes.data)
    kvd = KV * hd
    kc = rng.standard_normal((n_ctx, kvd)).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((n_ctx, kvd)).astype(np.float16).view(np.uint16)
    dkc, dvc = sa.DevBuf.of(kc), sa.DevBuf.of(vc)
    dcos, dsin = sa.DevBuf.of(cos_t), sa.DevBuf.of(sin_t)
    part = sa.DevBuf(sa.lib().sml_hip_attn_part_floats(H, hd, n_ctx) * 4)
    out = sa.DevBuf(H * hd * 4)
    oq = sa.Act(H * hd)
    scratch = np.zeros(n_ctx, np.float32)
    inv = np.float32(1) / np.sqrt(np.float32(hd))
    results = []
    for pos in positions:
        q = (rng.standard_normal(H * hd) * 2).astype(np.float32)
        k = (rng.standard_normal(kvd) * 2).astype(np.float32)
        v = rng.standard_normal(kvd).astype(np.float32)
        dq, dk, dv = sa.DevBuf.of(q), sa.DevBuf.of(k), sa.DevBuf.of(v)
        dpos = sa.DevBuf.of(np.array([pos], np.int32))
        sa.lib().sml_hip_set_exact(1 if exact else 0)
        try:
            if pos % 2:
                # odd positions: the launch that also quantizes its output for o
                rc = sa.lib().sml_hip_attention_q(dq.ptr, dk.ptr, dv.ptr, dkc.ptr, dvc.ptr, dcos.ptr, dsin.ptr,
                                                  dpos.ptr, H, KV, hd, n_ctx, part.ptr, out.ptr, oq.q.ptr,
                                                  oq.scale.ptr, oq.sums.ptr)
            else:
                rc = sa.lib().sml_hip_attention(dq.ptr, dk.ptr, dv.ptr, dkc.ptr, dvc.ptr, dcos.ptr, dsin.ptr,
                                                dpos.ptr, H, KV, hd, n_ctx, part.ptr, out.ptr)
        finally:
            sa.lib().sml_hip_set_exact(0)
        assert rc == 0, sa.lib().sml_hip_last_error()
        if pos % 2:
            got_out = out.read(np.float32)
            for a, b, name in zip(oq.read(), ob.quantize_act(got_out), ("q", "scale", "sums")):
                np.testing.assert_array_equal(a, b, err_msg=f"quantized attention output {name}, position {pos}")
        qr, kr = q.copy(), k.copy()
        ob.oracle().orc_rope(qr.ctypes.data, H, hd, half, cos_t[pos * half:].ctypes.data, sin_t[pos * half:].ctypes.data)
        ob.oracle().orc_rope(kr.ctypes.data, KV, hd, half, cos_t[pos * half:].ctypes.data, sin_t[pos * half:].ctypes.data)
        kc[pos] = kr.astype(np.float16).view(np.uint16)
        vc[pos] = v.astype(np.float16).view(np.uint16)
        got_k = dkc.read(np.uint16).reshape(n_ctx, kvd)[pos]
        got_v = dvc.read(np.uint16).reshape(n_ctx, kvd)[pos]
        np.testing.assert_array_equal(got_k, kc[pos], err_msg=f"K row {pos}")
        np.testing.assert_array_equal(got_v, vc[pos], err_msg=f"V row {pos}")
        want = np.zeros(H * hd, np.float32)
        for h in range(H):
            kh = h // (H // KV)
            ob.oracle().orc_attn_head(qr[h * hd:].ctypes.data, kc[:, kh * hd:].ctypes.data, vc[:, kh * hd:].ctypes.data,
                                      kvd, pos, hd, inv, scratch.ctypes.data, want[h * hd:].ctypes.data)
        results.append((pos, out.read(np.float32), want))
    return results


@pytest.mark.parametrize("heads", [(32, 8), (12, 2)])
def test_exact_attention_4096(heads):
    """At a 4096-position context, positions 0, 1, 2111, 2112 and 4095 (the
    last of the Llama-shaped workload): the rotated K row and the V row as
    stored, and the output of every head, equal the oracle's bit for bit."""
    for pos, got, want in attention_case(*heads, 4096, [0, 1, 2111, 2112, 4095], True, seed=heads[0]):
        same_bits(got, want, f"exact attention {heads} pos {pos}")


@pytest.mark.parametrize("split", ["64", "128"])
@pytest.mark.parametrize("heads", [(32, 8), (12, 2)])
def test_fast_attention_4096(heads, split, monkeypatch):
    """The decode path's split attention (splits of 64 or 128 positions,
    merged) at the same positions of a 4096-position context: K/V rows bit
    for bit, outputs within 1e-3 of the oracle (max |d| <= 1e-3 max |ref|,
    rel-RMS <= 1e-4)."""
    monkeypatch.setenv("SML_ATTN_CHUNK", split)
    for pos, got, want in attention_case(*heads, 4096, [0, 1, 2111, 2112, 4095], False, seed=heads[0] + 1):
        err = np.abs(got.astype(np.float64) - want)
        assert err.max() <= 1e-3 * np.abs(want).max(), (pos, err.max())
        assert np.sqrt((err ** 2).mean() / (want.astype(np.float64) ** 2).mean()) <= 1e-4, pos


@pytest.mark.parametrize("split", ["", "64"])
@pytest.mark.parametrize("heads", [(32, 8), (14, 2), (9, 3)])
def test_fast_attention_4096_head_dim_64(heads, split, monkeypatch):
    """head_dim 64 (the Llama-3.2-1B, Qwen2.5-0.5B and SmolLM shapes): a
    position's dims on 8 lanes, RoPE's partner lane i ^ 4, two positions per
    16-lane row combined before the row reductions. At positions 0, 1, 2111,
    2112 and 4095 of a 4096-position context: K/V rows bit for bit, outputs
    within 1e-3 of the oracle (max |d| <= 1e-3 max |ref|, rel-RMS <= 1e-4)."""
    if split:
        monkeypatch.setenv("SML_ATTN_CHUNK", split)
    for pos, got, want in attention_case(*heads, 4096, [0, 1, 2111, 2112, 4095], False, seed=heads[0] + 7, hd=64):
        err = np.abs(got.astype(np.float64) - want)
        assert err.max() <= 1e-3 * np.abs(want).max(), (pos, err.max())
        assert np.sqrt((err ** 2).mean() / (want.astype(np.float64) ** 2).mean()) <= 1e-4, pos


# ------------------------------------------------------------ the forward pass

DECODERS = {
    "dense": dict(n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000, qkv_bias=True,
                  random_perm=True, seed=31),
    "inorder": dict(n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000, qkv_bias=True,
                    random_perm=False, seed=32),
    "qwenish": dict(n_layer=4, n_embd=1536, n_head=12, n_head_kv=2, n_ff=8960, n_vocab=32000, rope_theta=1e6,
                    qkv_bias=True, tied=True, random_perm=True, seed=1002),
    "dense_q8": dict(n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000, qkv_bias=True,
                     random_perm=True, nbits=8, seed=33),
}
STARTS = {"dense": 11, "inorder": 7, "qwenish": 100, "dense_q8": 13}


@pytest.fixture(scope="module")
def decoder_file(tmp_path_factory):
    made = {}

    def get(name):
        if name not in made:
            p = tmp_path_factory.mktemp("xdec") / f"{name}.ssf"
            sa.synth_model(p, **DECODERS[name])
            made[name] = p
        return made[name]
    return get


@needs_ref
@pytest.mark.parametrize("name", list(DECODERS))
def test_exact_teacher_forced_equals_reference(decoder_file, name):
    """Teacher-forced on 32 random ids, every logit of every step equals the
    reference's sml_forward bit for bit (Qwen-shaped layers with q/k/v bias,
    a tied 32000-token head, permuted and in-order inputs)."""
    p = decoder_file(name)
    V = DECODERS[name]["n_vocab"]
    ids = np.random.default_rng(5).integers(0, V, 32)
    d = sa.Decoder(p, n_ctx=64, exact=True)
    rm = ob.RefModel(p, 64, threads=min(16, os.cpu_count() or 1))
    try:
        assert d.exact
        for pos, tok in enumerate(ids):
            same_bits(d.step(int(tok), pos, V), rm.forward(int(tok), pos), f"{name} position {pos}")
    finally:
        d.close()
        rm.close()


@needs_ref
@pytest.mark.parametrize("name", list(DECODERS))
def test_exact_greedy_64_equals_reference(decoder_file, name):
    """64 free-running greedy tokens (one captured graph per token, the
    argmax fed back on the device) are the reference's 64 greedy tokens, and
    those take at least 8 distinct ids."""
    p = decoder_file(name)
    start, n = STARTS[name], 64
    d = sa.Decoder(p, n_ctx=128, exact=True)
    try:
        gpu = [int(t) for t in d.generate(start, 0, n)]
    finally:
        d.close()
    rm = ob.RefModel(p, 128, threads=min(16, os.cpu_count() or 1))
    ref, tok = [], start
    try:
        for pos in range(n):
            tok = int(np.argmax(rm.forward(tok, pos)))
            ref.append(tok)
    finally:
        rm.close()
    assert len(set(ref)) >= 8, f"the reference's greedy ids are not diverse: {ref}"
    first = next((i for i, (a, b) in enumerate(zip(gpu, ref)) if a != b), None)
    assert first is None, f"step {first}: gpu {gpu[first]} reference {ref[first]}"


@needs_ref
@pytest.mark.parametrize("name,n", [("dense", 130), ("inorder", 64), ("qwenish", 77), ("dense_q8", 100)])
def test_exact_batched_prompt_equals_reference(decoder_file, name, n):
    """Exact mode reads a prompt batched (level 1: 64-position chunks through
    the reference-order Q4 or Q8 GEMM, sml_xgemm_q4 / _q8, and the row form
    of the reference-order attention), and its logits equal the reference
    stepping the same ids through sml_forward bit for bit; so do 4 greedy
    steps after it. Chunk boundaries inside the prompt (130 = 64 + 64 + 2),
    one whole chunk (64), Qwen-shaped layers (77), Q8 layers (100). The same
    prompt read a token at a time (level 0) gives the same bits."""
    p = decoder_file(name)
    V = DECODERS[name]["n_vocab"]
    ids = np.random.default_rng(n).integers(0, V, n).astype(np.int32)
    rm = ob.RefModel(p, 256, threads=min(16, os.cpu_count() or 1))
    try:
        for pos, tok in enumerate(ids):
            want = rm.forward(int(tok), pos)
        wants, toks = [want], [int(np.argmax(want))]
        for i in range(4):
            wants.append(rm.forward(toks[-1], n + i))
            toks.append(int(np.argmax(wants[-1])))
    finally:
        rm.close()
    for level in (1, 0):
        d = sa.Decoder(p, n_ctx=256, exact=True)
        try:
            assert d.exact
            d.prompt_mode(level)
            got = [d.prefill(ids, 0, V)]
            for i in range(4):
                got.append(d.step(toks[i], n + i, V))
        finally:
            d.close()
        for i, (g, w) in enumerate(zip(got, wants)):
            same_bits(g, w, f"{name} level {level} {'prompt' if i == 0 else f'step {i}'}")
