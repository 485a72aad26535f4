"""Ingest on the GPU: the quantizer's searches, the GPTQ/AWQ unpacker and the
whole re-quantization into SSF planes, against the reference quantizer's own
C library (oracle/_ref/libsmlquant.so, built from sml/sml-quant.c) and the
oracle's restatement, bit for bit; then the re-quantized matrix through the
GEMV and an SSF file read back by the library's loader."""
import ctypes

import numpy as np
import pytest

import sheep_amd as sa
from oracle import bind as ob
from sheep_amd import gptq, ingest

pytestmark = pytest.mark.gpu
needs_refq = pytest.mark.skipif(not ob.have_refq(), reason="the reference quantizer's library was not built here")


def _data(rng, rows, cols):
    w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.02
    w[1, :64] = 0.25                                   # constant groups
    w[2, 96:128] = 0.0
    lv = ((rng.integers(0, 16, (rows, cols)) - 8) * 0.01).astype(np.float16).astype(np.float32)
    return {"normal": w, "levels": lv}


@needs_refq
@pytest.mark.parametrize("group", [32, 64])
@pytest.mark.parametrize("weighted", [False, True])
def test_asym_grid_dropin_equals_reference_library(group, weighted):
    # the library's sml_asym_grid, bound with the reference loader's argument
    # types, against the reference's own build of sml-quant.c
    rng = np.random.default_rng(100 + group + weighted)
    rows, cols = 96, 2048
    wt = (rng.random(cols).astype(np.float32) ** 2 + np.float32(0.1)) if weighted else None
    for name, w in _data(rng, rows, cols).items():
        for target in (None, 3):
            print(f"asym_grid {name} group {group} weighted {weighted} target {target}", flush=True)
            kw = dict(rem=0 if target is None else 1, refit=1 if target is None else 0)
            lg, sg = ob.asym_grid(w, group, 4, wt, lib=ingest._lib(), **kw)
            lr, sr = ob.asym_grid(w, group, 4, wt, lib=ob.refq(), **kw)
            assert np.array_equal(lg.view(np.uint32), lr.view(np.uint32)), name
            assert np.array_equal(sg.view(np.uint32), sr.view(np.uint32)), name


@needs_refq
@pytest.mark.parametrize("weighted", [False, True])
def test_field_search_dropin_equals_reference_library(weighted):
    rng = np.random.default_rng(7)
    rows, cols = 64, 2048
    gps = 8
    wt = (rng.random(cols).astype(np.float32) + np.float32(0.5)) if weighted else None
    for name, w in _data(rng, rows, cols).items():
        lo, st = ob.asym_grid(w, 32, 4)
        d16, q8, _ = ob.two_level(st, gps, signed=False)
        md16, mq8, _ = ob.two_level(lo, gps, signed=True)
        print(f"field_search {name} weighted {weighted}", flush=True)
        dv = np.repeat(d16.view(np.float16).astype(np.float32), gps, axis=1)
        dm = np.repeat(md16.view(np.float16).astype(np.float32), gps, axis=1)
        gq, gm = ob.field_search(w, dv, dm, q8, mq8, 32, 15, wt=wt, radius=2, lib=ingest._lib())
        rq, rm = ob.field_search(w, dv, dm, q8, mq8, 32, 15, wt=wt, radius=2, lib=ob.refq())
        assert np.array_equal(gq, rq) and np.array_equal(gm, rm), name


def test_the_reference_prototypes_bind_and_agree():
    # sml_asym_grid / sml_field_search with the argument types the reference's
    # loader gives them (tooling/sml_grid_c.py:23-28)
    rng = np.random.default_rng(3)
    w = rng.standard_normal((16, 512)).astype(np.float32)
    facs = ob.grid_facs()
    l = ingest._lib()
    a_l, a_s = np.zeros((16, 16), np.float32), np.zeros((16, 16), np.float32)
    l.sml_asym_grid(w.ctypes.data, 16, 512, 32, 4, 0, None, facs.ctypes.data, len(facs), 3, 1, a_l.ctypes.data,
                    a_s.ctypes.data)
    b_l, b_s = ob.asym_grid(w, 32, 4)
    assert np.array_equal(a_l, b_l) and np.array_equal(a_s, b_s)
    # a refused shape prints its reason and leaves NaN, as the void prototype can
    l.sml_asym_grid(w.ctypes.data, 16, 500, 32, 4, 0, None, facs.ctypes.data, len(facs), 3, 1, a_l.ctypes.data,
                    a_s.ctypes.data)
    assert np.isnan(a_l.ravel()[:16 * (500 // 32)]).all()
    assert l.sml_hip_asym_grid(w.ctypes.data, 16, 500, 32, 4, 0, None, facs.ctypes.data, len(facs), 3, 1,
                               a_l.ctypes.data, a_s.ctypes.data) == -1
    assert b"groups must be" in sa.lib().sml_hip_last_error()


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_unpack_dequant_equals_oracle(bits):
    rng = np.random.default_rng(bits)
    rows, cols, group = 512, 2048, 128
    n = 1 << bits
    codes = rng.integers(0, n, (rows, cols))
    zeros = rng.integers(1, n, (rows, cols // group))
    scales = (np.abs(rng.standard_normal((rows, cols // group))) * 0.01 + 1e-3).astype(np.float16)
    for zero_add in (0, 1):
        qw, qz, sc = ingest.pack_gptq(codes, zeros, scales, bits, zero_add)
        for g_idx in (None, rng.permutation(np.arange(cols) // group).astype(np.int32)):
            print(f"unpack_dequant {bits} bits zero_add {zero_add} g_idx {g_idx is not None}", flush=True)
            t = {"qweight": qw, "qzeros": qz, "scales": sc, "g_idx": g_idx}
            qc = {"bits": bits, "group_size": group, "desc_act": g_idx is not None,
                  "checkpoint_format": "gptq" if zero_add else "gptq_v2"}
            got = ingest.dequant_gptq(t, qc)
            want = ob.unpack_dequant_f16(qw, qz, sc, g_idx, rows, cols, bits, group, zero_add)
            assert np.array_equal(got.astype(np.float32), want)


def test_unpack_dequant_awq_equals_oracle():
    rng = np.random.default_rng(44)
    rows, cols, group = 512, 2048, 128
    codes = rng.integers(0, 16, (rows, cols))
    zeros = rng.integers(0, 16, (rows, cols // group))
    scales = (np.abs(rng.standard_normal((rows, cols // group))) * 0.01 + 1e-3).astype(np.float16)
    for with_zeros in (True, False):
        qw, qz, sc = gptq.pack_awq(codes, zeros if with_zeros else None, scales)
        got = ingest.dequant_awq({"qweight": qw, "qzeros": qz, "scales": sc}, {"bits": 4, "group_size": group})
        want = ob.unpack_dequant_f16(qw, qz, sc, None, rows, cols, 4, group, awq=True)
        assert np.array_equal(got.astype(np.float32), want)


def _same(res, want, nbits):
    h = res.host()
    for k in ("sd", "sq", "md", "mq", "perm", "codes"):
        assert np.array_equal(h[k], want[k]), k
    # the packed planes unpack, through the oracle's reader, to the same codes
    v = ob.FlatView(h["planes"], h["sd"], h["md"], h["sq"], h["mq"], res.rows, res.cols, nbits)
    for r in (0, res.rows // 2, res.rows - 1):
        assert np.array_equal(v.codes(r), want["codes"][r]), r
    return h


@pytest.mark.parametrize("nbits", [2, 3, 4, 5, 6, 7, 8])
def test_requant_equals_oracle_every_width(nbits):
    rng = np.random.default_rng(300 + nbits)
    rows, cols = 128, 1024
    w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.02
    w[5, 256:512] = 0.0
    print(f"requant width {nbits}", flush=True)
    res = ingest.requantize(w, nbits, keep_codes=True)
    _same(res, ob.requant(w, nbits), nbits)


def test_requant_given_order_weights_and_radius():
    rng = np.random.default_rng(8)
    rows, cols = 64, 2048
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    perm = rng.permutation(cols).astype(np.int32)
    wt = (rng.random(cols).astype(np.float32) + 0.5)
    for radius in (0, 1, 2):
        print(f"requant perm given, radius {radius}", flush=True)
        res = ingest.requantize(w, 4, perm=perm, wt=wt, radius=radius, keep_codes=True)
        _same(res, ob.requant(w, 4, perm=perm, wt=wt, radius=radius), 4)


def test_ingest_gptq_at_the_width_sweep_shape():
    # the GPTQ-4 layout of the width sweep (4096 x 14336, group 128) re-quantized
    # to SSF Q4 on the device: equal to the oracle fed the same float16 copy,
    # and its GEMV within the quantization error of the GPTQ GEMV
    rows, cols = 4096, 14336
    qw, qz, sc = gptq.synth(rows, cols, 1004)
    t = {"qweight": qw, "qzeros": qz, "scales": sc}
    qc = {"bits": 4, "group_size": 128}
    print("ingest_gptq 4096x14336", flush=True)
    res = ingest.ingest_gptq(t, qc, keep_codes=True)
    w16 = ob.unpack_dequant_f16(qw, qz, sc, None, rows, cols, 4, 128, 1)
    want = ob.requant(w16, 4)
    h = _same(res, want, 4)
    print(f"re-quantized in {res.ms:.2f} ms of GPU time", flush=True)
    x = np.random.default_rng(5).standard_normal(cols).astype(np.float32)
    m = res.mat()
    xd = sa.DevBuf.of(x[h["perm"]])
    act, y = sa.Act(cols), sa.DevBuf(rows * 4)
    sa.normq(xd, act)
    sa.matvec(m, act, y)
    got = y.read(np.float32)
    ref = w16.astype(np.float64) @ x.astype(np.float64)
    rel = np.sqrt(np.mean((got - ref) ** 2) / np.mean(ref ** 2))
    print(f"re-quantized GEMV vs the float16 copy: rel-RMS {rel:.4f}", flush=True)
    # the format's own loss on this recipe: two GPTQ groups of independent
    # scales share each superblock's 8-bit step and min fields, so the smaller
    # group's levels are coarse; the oracle reproduces the same fields exactly
    assert rel < 0.1
    # the oracle's GEMV on the same planes and activation
    q, s, u = act.read()
    v = ob.FlatView(h["planes"], h["sd"], h["md"], h["sq"], h["mq"], rows, cols, 4)
    yo = v.matvec(q, s, u)
    assert np.abs(got - yo).max() <= 1e-3 * np.abs(yo).max()


def test_ingest_awq_and_written_file(tmpdir_s):
    rng = np.random.default_rng(12)
    rows, cols, group = 1024, 4096, 128
    codes = rng.integers(0, 16, (rows, cols))
    zeros = rng.integers(0, 16, (rows, cols // group))
    scales = (np.abs(rng.standard_normal((rows, cols // group))) * 0.002 + 1e-4).astype(np.float16)
    qw, qz, sc = gptq.pack_awq(codes, zeros, scales)
    res = ingest.ingest_awq({"qweight": qw, "qzeros": qz, "scales": sc}, {"bits": 4, "group_size": group},
                            keep_codes=True)
    w16 = ob.unpack_dequant_f16(qw, qz, sc, None, rows, cols, 4, group, awq=True)
    h = _same(res, ob.requant(w16, 4), 4)
    path = tmpdir_s / "awq_ingest.ssf"
    res.write_ssf(path, "blk.0.ffn_up.weight")
    m = sa.Mat.from_file(path, "blk.0.ffn_up.weight")
    assert np.array_equal(sa.unpack(m, 0, rows), h["codes"])
    from sheep_amd import ssf
    t = ssf.SSF(path)["blk.0.ffn_up.weight"]
    assert np.array_equal(t.perm, h["perm"])
    if ob.have_ref():
        for r in (0, 511, 1023):
            assert np.array_equal(ob.ref_dequant_row(t, r), ob.dequant_row(t, r))


def _gguf_blocks(kind, rows, cols, rng):
    """Random GGUF blocks of one type: random code bytes; fp16 d of assorted
    sizes, a few zero, subnormal or negative."""
    gtype, qk, bs, _ = ingest.GGUF_TYPES[kind]
    b = rng.integers(0, 256, (rows, cols // qk, bs)).astype(np.uint8)
    d = (rng.standard_normal((rows, cols // qk)) * 0.02).astype(np.float16)
    d.flat[::97] = np.float16(0)
    d.flat[5::89] = np.float16(3e-7)                  # subnormal in fp16
    at = 208 if kind == "Q6_K" else 0
    b[..., at:at + 2] = d[..., None].view(np.uint8)
    return gtype, b


@pytest.mark.parametrize("kind", ["Q8_0", "Q4_0", "Q6_K"])
def test_gguf_dequant_equals_oracle(kind):
    """Every weight of the device's float16 copy equals the oracle's
    restatement of ggml's dequantize_row_* bit for bit."""
    rng = np.random.default_rng(len(kind) * 31 + ord(kind[1]))
    rows, cols = 300, 4096
    gtype, b = _gguf_blocks(kind, rows, cols, rng)
    got = ingest.gguf_dequant(kind, b, rows, cols).read(np.float32).reshape(rows, cols)
    want = ob.gguf_dequant_f16(gtype, b, rows, cols)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("kind", ["Q8_0", "Q6_K", "Q4_0"])
def test_ingest_gguf_equals_oracle(kind):
    """A GGUF tensor of each type re-quantized at the type's own width (8,
    6, 4 bits): fields, order and codes equal the oracle's re-quantization of
    the oracle's float16 copy, and its GEMV stays within the re-quantization
    error of that copy."""
    rng = np.random.default_rng(90 + len(kind))
    rows, cols = 512, 2048
    gtype, b = _gguf_blocks(kind, rows, cols, rng)
    nb = ingest.GGUF_TYPES[kind][3]
    print(f"ingest_gguf {kind} {rows}x{cols} -> Q{nb}", flush=True)
    res = ingest.ingest_gguf(kind, b, rows, cols, keep_codes=True)
    w16 = ob.gguf_dequant_f16(gtype, b, rows, cols)
    h = _same(res, ob.requant(w16, nb), nb)
    x = np.random.default_rng(3).standard_normal(cols).astype(np.float32)
    xd = sa.DevBuf.of(x[h["perm"]])
    act, y = sa.Act(cols), sa.DevBuf(rows * 4)
    sa.normq(xd, act)
    sa.matvec(res.mat(), act, y)
    got = y.read(np.float32)
    ref = w16.astype(np.float64) @ x.astype(np.float64)
    rel = np.sqrt(np.mean((got - ref) ** 2) / np.mean(ref ** 2))
    print(f"{kind}: re-quantized GEMV vs the float16 copy rel-RMS {rel:.4f}", flush=True)
    assert rel < 0.1
