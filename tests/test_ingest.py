"""Re-quantization of GPTQ/AWQ copies into SSF planes (the ingest path): the
oracle's restatement pinned against the reference quantizer's own C library
(sml/sml-quant.c, built from its source into oracle/_ref), numpy's linspace,
hand-worked known answers, a round trip through representable tensors, and
the reference engine's own dequantizers reading the written file.
"""
import numpy as np
import pytest

import sheep_amd as sa
from oracle import bind as ob
from sheep_amd import ingest

needs_refq = pytest.mark.skipif(not ob.have_refq(), reason="the reference quantizer's sources are not present")
needs_ref = pytest.mark.skipif(not ob.have_ref(), reason="the reference engine's sources are not present")


def tensors(rng, rows, cols):
    """The kinds of data the searches meet: gaussian weights, uniform ones, a
    float16 copy of a 4-bit GPTQ tensor (discrete levels), and groups that are
    constant or zero."""
    out = {"normal": rng.standard_normal((rows, cols)).astype(np.float32) * 0.02,
           "uniform": rng.uniform(-1, 1, (rows, cols)).astype(np.float32),
           "levels": ((rng.integers(0, 16, (rows, cols)) - 8) * 0.01).astype(np.float16).astype(np.float32)}
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    w[:, :32] = 0.5
    w[3, 64:96] = 0.0
    out["flat_groups"] = w
    return out


def test_grid_factors_are_numpys_linspace():
    # tooling/sml_grid_c.py:41-42 builds them with numpy, which is what pins them
    for ncand in (20, 12, 6, 3):
        want = np.concatenate([np.linspace(0.6, 0.85, max(2, ncand // 3)),
                               np.linspace(0.88, 1.04, max(2, ncand - ncand // 3))]).astype(np.float32)
        assert np.array_equal(ob.grid_facs(ncand), want)


@needs_refq
@pytest.mark.parametrize("group", [32, 64, 8])
@pytest.mark.parametrize("weighted", [False, True])
def test_asym_grid_equals_reference_library(group, weighted):
    rng = np.random.default_rng(7 + group)
    rows, cols = 24, 1024
    wt = None
    if weighted:
        imp = rng.random(cols).astype(np.float32) ** 2 + 0.1
        wt = imp / max(float(imp.mean()), 1e-30) + np.float32(1e-6)
    for name, w in tensors(rng, rows, cols).items():
        for rem, refit in ((0, 1), (1, 0), (0, 0)):
            lo, so = ob.asym_grid(w, group, 4, wt, rem=rem, refit=refit)
            lr, sr = ob.asym_grid(w, group, 4, wt, rem=rem, refit=refit, lib=ob.refq())
            assert np.array_equal(lo.view(np.uint32), lr.view(np.uint32)), (name, rem)
            assert np.array_equal(so.view(np.uint32), sr.view(np.uint32)), (name, rem)


@needs_refq
@pytest.mark.parametrize("weighted", [False, True])
def test_field_search_equals_reference_library(weighted):
    rng = np.random.default_rng(11)
    rows, cols = 24, 1024
    ng = cols // 32
    wt = None if not weighted else rng.random(cols).astype(np.float32) + 0.5
    for name, w in tensors(rng, rows, cols).items():
        dv = np.abs(rng.standard_normal((rows, ng))).astype(np.float32) * 0.001
        dm = np.abs(rng.standard_normal((rows, ng))).astype(np.float32) * 0.001
        dv[0, :4] = 0.0
        q8 = rng.integers(1, 256, (rows, ng)).astype(np.int32)
        m8 = rng.integers(0, 255, (rows, ng)).astype(np.int32)
        for radius in (0, 1, 2):
            a = ob.field_search(w, dv, dm, q8, m8, 32, 15, radius=radius, wt=wt)
            b = ob.field_search(w, dv, dm, q8, m8, 32, 15, radius=radius, wt=wt, lib=ob.refq())
            assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), (name, radius)


def test_grid_recovers_an_exact_grid():
    # every group exactly on a 16-level grid with both end codes used: the
    # refitted grid reconstructs it to float rounding
    rng = np.random.default_rng(3)
    rows, cols = 8, 512
    codes = rng.integers(0, 16, (rows, cols))
    codes[:, ::32] = 0
    codes[:, 1::32] = 15
    step = np.repeat(np.abs(rng.standard_normal((rows, cols // 32))) * 0.01 + 1e-3, 32, axis=1)
    mins = np.repeat(-rng.random((rows, cols // 32)) * 0.1, 32, axis=1)
    w = (codes * step + mins).astype(np.float32)
    lo, so = ob.asym_grid(w, 32, 4)
    L, S = np.repeat(lo, 32, axis=1), np.repeat(so, 32, axis=1)
    c = np.clip(np.rint((w - L) / S), 0, 15)
    assert np.array_equal(c, codes)
    assert np.max(np.abs(c * S + L - w)) <= 1e-6 * np.max(np.abs(w))


def test_two_level_known_answers():
    # steps: superblock maximum 2.55 -> d = f16(2.55/255) = f16(0.01) =
    # 2^-7 * (1 + 287/1024) = 0.01000213623046875
    v = np.array([[2.55, 1.0, 0.5, 0.0, 2.5, 0.01, 1.275, 0.3]], np.float32)
    d16, q8, eff = ob.two_level(v, signed=False)
    d = np.float32(0.01000213623046875)
    assert d16[0, 0] == 0x2000 | 287
    # 2.55/d = 254.95 -> 255; 1.0/d = 99.98 -> 100; 0 -> clipped up to 1;
    # 0.01/d = 0.9998 -> 1; 1.275/d = 127.47 -> 127
    assert list(q8[0]) == [255, 100, 50, 1, 250, 1, 127, 30]
    assert eff[0, 1] == np.float32(100) * d
    # mins: maximum |v| 1.27 -> md = f16(0.01); stored biased by 127, clipped to 0..254
    m = np.array([[-1.27, 0.0, 0.5, -0.33, 1.27, 0.004, -0.006, 0.1]], np.float32)
    md16, mq8, em = ob.two_level(m, signed=True)
    dm = d                                   # f16(1.27/127) is the same fp16 value
    assert md16[0, 0] == 0x2000 | 287
    # -1.27/d = -126.97 -> -127 -> 0; 0.5/d = 49.99 -> 177; -0.33/d = -32.99 -> 94;
    # 0.004/d = 0.40 -> 127; -0.006/d = -0.60 -> 126; 0.1/d = 9.998 -> 137
    assert list(mq8[0]) == [0, 127, 177, 94, 254, 127, 126, 137]
    assert em[0, 0] == (np.float32(0) - 127) * dm
    # an all-zero superblock divides by 1e-8 and stores d = 0
    z16, zq, _ = ob.two_level(np.zeros((1, 8), np.float32), signed=True)
    assert z16[0, 0] == 0 and np.all(zq == 127)


def test_two_level_bounds():
    rng = np.random.default_rng(5)
    # values whose scales are normal fp16 numbers (below about 6e-5 * 255 the
    # scale is an fp16 subnormal, rounded coarsely, and the top codes clip)
    v = np.abs(rng.standard_normal((64, 128))).astype(np.float32)
    d16, q8, eff = ob.two_level(v, signed=False)
    d = np.repeat(d16.view(np.float16).astype(np.float32), 8, axis=1)
    assert q8.min() >= 1
    ok = v >= d   # values above the floor of one level round to within half a level
    assert np.all(np.abs(eff - v)[ok] <= 0.5 * d[ok] * (1 + 1e-6))
    m = rng.standard_normal((64, 128)).astype(np.float32)
    md16, mq8, em = ob.two_level(m, signed=True)
    dm = np.repeat(md16.view(np.float16).astype(np.float32), 8, axis=1)
    assert mq8.max() <= 254
    inside = np.abs(m) <= 127 * dm
    assert np.all(np.abs(em - m)[inside] <= 0.5 * dm[inside] * (1 + 1e-6))
    # subnormal scales: the codes stay in range and the largest value clips to the top code
    t16, tq, _ = ob.two_level(v * 1e-3, signed=False)
    assert tq.min() >= 1 and tq.max() == 255


def test_perm_is_a_stable_ascending_order_of_the_column_maximum():
    rng = np.random.default_rng(9)
    w = ((rng.integers(0, 16, (64, 512)) - 8) * 0.01).astype(np.float16).astype(np.float32)   # many ties
    w[:, 7] = np.nan
    p = ob.perm_maxabs(w)
    key = np.abs(w).max(axis=0)
    key = np.where(np.isnan(np.abs(w)).any(axis=0), np.inf, key)      # NaN keys last
    want = np.lexsort((np.arange(512), key))
    assert np.array_equal(p, want)
    assert len(set(p.tolist())) == 512 and p[-1] == 7


def _gptq_case(rng, rows, cols, bits, group, zero_add):
    n = 1 << bits
    codes = rng.integers(0, n, (rows, cols))
    zeros = rng.integers(1, n, (rows, cols // group))
    scales = (np.abs(rng.standard_normal((rows, cols // group))) * 0.01 + 1e-3).astype(np.float16)
    qw, qz, sc = ingest.pack_gptq(codes, zeros, scales, bits, zero_add)
    return codes, zeros, scales, qw, qz, sc


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("zero_add", [0, 1])
def test_unpack_dequant_known_answer(bits, zero_add):
    # integers chosen, packed, unpacked: (code - zero) * scale in fp32, then float16
    rng = np.random.default_rng(bits * 10 + zero_add)
    rows, cols, group = 64, 256, 64
    codes, zeros, scales, qw, qz, sc = _gptq_case(rng, rows, cols, bits, group, zero_add)
    got = ob.unpack_dequant_f16(qw, qz, sc, None, rows, cols, bits, group, zero_add)
    g = np.arange(cols) // group
    want = ((codes - zeros[:, g]).astype(np.float32) * scales[:, g].astype(np.float32)).astype(np.float16)
    assert np.array_equal(got, want.astype(np.float32))


def test_unpack_dequant_g_idx_and_awq():
    rng = np.random.default_rng(21)
    rows, cols, group = 64, 512, 128
    codes, zeros, scales, qw, qz, sc = _gptq_case(rng, rows, cols, 4, group, 1)
    g_idx = rng.permutation(np.arange(cols) // group).astype(np.int32)
    got = ob.unpack_dequant_f16(qw, qz, sc, g_idx, rows, cols, 4, group, 1)
    want = ((codes - zeros[:, g_idx]).astype(np.float32) * scales[:, g_idx].astype(np.float32)).astype(np.float16)
    assert np.array_equal(got, want.astype(np.float32))
    # the same through the 4-bit oracle the GPTQ GEMV is pinned by, rounded to fp16
    row = np.zeros(cols, np.float32)
    o = ob.oracle()
    o.orc_gptq_dequant_row_gidx(qw.ctypes.data, qz.ctypes.data, sc.view(np.uint16).ctypes.data, g_idx.ctypes.data,
                                rows, cols, group, 1, 5, row.ctypes.data)
    assert np.array_equal(got[5], row.astype(np.float16).astype(np.float32))
    # AWQ: the output nibble order and the default zero of 8
    from sheep_amd import gptq
    for with_zeros in (True, False):
        z = zeros if with_zeros else np.full_like(zeros, 8)
        aqw, aqz, asc = gptq.pack_awq(codes, z if with_zeros else None, scales)
        got = ob.unpack_dequant_f16(aqw, aqz, asc, None, rows, cols, 4, group, awq=True)
        g = np.arange(cols) // group
        want = ((codes - z[:, g]).astype(np.float32) * scales[:, g].astype(np.float32)).astype(np.float16)
        assert np.array_equal(got, want.astype(np.float32))


def representable(rng, rows, cols, nbits):
    """An SSF FLAT tensor whose every superblock holds a group with step field
    255 and one with min field 0 (so the two-level scales are recovered), and
    whose every group uses both end codes: (codes, sd, sq, md, mq)."""
    ng, ns, n = cols // 32, cols // 256, (1 << nbits) - 1
    codes = rng.integers(0, n + 1, (rows, cols)).astype(np.uint8)
    codes[:, ::32] = 0
    codes[:, 1::32] = n
    sd = (np.abs(rng.standard_normal((rows, ns))) * 1e-4 + 2e-5).astype(np.float16)
    md = (np.abs(rng.standard_normal((rows, ns))) * 1e-3 + 1e-4).astype(np.float16)
    sq = rng.integers(60, 256, (rows, ng)).astype(np.uint8)
    mq = rng.integers(0, 127, (rows, ng)).astype(np.uint8)
    sq[:, ::8] = 255
    mq[:, 1::8] = 0
    return codes, sd.view(np.uint16), sq, md.view(np.uint16), mq


def dequant(codes, sd, sq, md, mq):
    """code*step + min with step = f16(sd)*sq, min = f16(md)*(mq - 127), in fp32."""
    step = np.repeat(sd.view(np.float16).astype(np.float32), 8, axis=1) * sq.astype(np.float32)
    mn = np.repeat(md.view(np.float16).astype(np.float32), 8, axis=1) * (mq.astype(np.float32) - np.float32(127))
    return codes.astype(np.float32) * np.repeat(step, 32, axis=1) + np.repeat(mn, 32, axis=1)


@pytest.mark.parametrize("nbits", [2, 4, 8])
def test_requant_of_a_representable_tensor_is_the_identity(nbits):
    rng = np.random.default_rng(40 + nbits)
    rows, cols = 16, 512
    codes, sd, sq, md, mq = representable(rng, rows, cols, nbits)
    w = dequant(codes, sd, sq, md, mq)
    ident = np.arange(cols, dtype=np.int32)
    r = ob.requant(w, nbits, perm=ident)
    assert np.array_equal(r["codes"], codes)
    assert np.array_equal(r["sd"], sd) and np.array_equal(r["md"], md)
    assert np.array_equal(r["sq"], sq) and np.array_equal(r["mq"], mq)
    assert np.array_equal(r["perm"], ident)


def test_requant_error_is_a_fraction_of_a_level():
    rng = np.random.default_rng(12)
    rows, cols = 32, 1024
    w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.02
    r = ob.requant(w, 4)
    wp = w[:, r["perm"]]
    back = dequant(r["codes"], r["sd"], r["sq"], r["md"], r["mq"])
    step = np.repeat(np.repeat(r["sd"].view(np.float16).astype(np.float32), 8, axis=1) * r["sq"], 32, axis=1)
    err = np.abs(back - wp)
    # the grid may clip a few outliers; the rest round to within half a level
    assert np.mean(err <= 0.5 * step * (1 + 1e-5)) > 0.98
    assert np.sqrt(np.mean(err ** 2)) / np.sqrt(np.mean(wp ** 2)) < 0.1


def pack_planes(codes, nbits):
    """The FLAT planes of `codes` [rows][cols] per tooling/sml_format.py:392-448
    (nibbles in 64-byte quads, 2-bit group-planar, 1-bit LSB first) and the
    plane order of tooling/sml_quantize.py:104-106,614-651."""
    rows, cols = codes.shape
    c = codes.astype(np.uint8)
    order = {2: [(2, 0)], 3: [(2, 0), (1, 2)], 4: [(4, 0)], 5: [(4, 0), (1, 4)], 6: [(2, 4), (4, 0)],
             7: [(4, 0), (2, 4), (1, 6)], 8: [(4, 0), (4, 4)]}[nbits]
    out = []
    for bits, shift in order:
        part = (c >> shift) & ((1 << bits) - 1)
        if bits == 4:
            q = part.reshape(rows, cols // 128, 4, 32)
            pl = np.concatenate([q[:, :, 0] | (q[:, :, 1] << 4), q[:, :, 2] | (q[:, :, 3] << 4)], axis=2)
        elif bits == 2:
            q = part.reshape(rows, cols // 128, 4, 32)
            pl = q[:, :, 0] | (q[:, :, 1] << 2) | (q[:, :, 2] << 4) | (q[:, :, 3] << 6)
        else:
            pl = np.packbits(part.reshape(rows, cols // 8, 8), axis=2, bitorder="little")
        out.append(np.ascontiguousarray(pl.reshape(rows, -1).astype(np.uint8)))
    return out


@needs_ref
@pytest.mark.parametrize("nbits", [2, 3, 4, 5, 6, 7, 8])
def test_written_file_reads_back_through_the_reference(tmpdir_s, nbits):
    # the writer's layout read by the repository's reader, the oracle's
    # unpacker and the reference engine's own dequantizers
    import ctypes
    from sheep_amd import ssf
    rng = np.random.default_rng(60 + nbits)
    rows, cols = 8, 512
    codes, sd, sq, md, mq = representable(rng, rows, cols, nbits)
    perm = rng.permutation(cols).astype(np.int32)
    planes = pack_planes(codes, nbits)
    path = str(tmpdir_s / f"ingest_q{nbits}.ssf")
    pl = (ctypes.c_void_p * 3)(*([p.ctypes.data for p in planes] + [None] * (3 - len(planes))))
    assert ingest._lib().sml_hip_ssf_write_quant(path.encode(), b"blk.0.ffn_up.weight", rows, cols, nbits, pl,
                                                 sd.ctypes.data, sq.ctypes.data, md.ctypes.data, mq.ctypes.data,
                                                 perm.ctypes.data) == 0
    t = ssf.SSF(path)["blk.0.ffn_up.weight"]
    assert np.array_equal(t.perm, perm)
    back = dequant(codes, sd, sq, md, mq)
    for r in range(rows):
        assert np.array_equal(ob.unpack(t, r), codes[r])
        got = ob.ref_dequant_row(t, r)
        # the reference's dequantizers per width (some fuse code*step + min)
        assert np.array_equal(got, ob.dequant_row(t, r)), r
        assert np.allclose(got, back[r], rtol=1e-6, atol=0), r
