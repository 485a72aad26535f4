"""GGUF Q4_K and Q5_K blocks (ggml's block_q4_K, block_q5_K) repacked into
the FLAT Q4 and Q5 layouts.

The reference reads GGUF only through transformers into fp16, then
re-quantizes (tooling/sml_gguf.py:1-35), and `gguf` is not importable here;
the blocks are pinned instead by ggml's published format: hand-built blocks
with known answers, the quantizer's scale packing as a round trip, and the
oracle's restatement of dequantize_row_q4_K (orc_q4k_dequant_row). A Q4_K
weight d*sc*q - dmin*m is the FLAT record's step*q + min with sd = d, sq = sc,
md = dmin, mq = 127 - m, and the 128 code bytes are already FLAT quads, so the
repack (sml_hip_q4k_repack) moves bytes and fields only: after it the SSF
dequantization equals the published formula bit for bit, and the GPU's codes
are the block's nibbles. Q5_K adds a fifth code bit per weight (qh: bit j of
byte l for weight l of sub-block j) to the same fields and nibbles; it
becomes the FLAT Q5 record's 1-bit plane, pinned the same way against
dequantize_row_q5_K (orc_q5k_dequant_row).
"""
import numpy as np
import pytest

import sheep_amd as sa
from oracle import bind as ob


def known_block():
    """d = 1, dmin = 0.5, sub-block j: scale j+1, min j; weight i has code i % 16."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.5], np.float16).view(np.uint8)
    blk[4:16] = ob.q4k_pack_scales([1, 2, 3, 4, 5, 6, 7, 8], [0, 1, 2, 3, 4, 5, 6, 7])
    l = np.arange(32) % 16
    for c in range(4):
        blk[16 + 32 * c:16 + 32 * (c + 1)] = l | (l << 4)
    return blk


def test_q4k_known_answers():
    """Values worked out by hand from the format's definition."""
    w = ob.q4k_dequant(known_block(), 1, 256)[0]
    # (index, sub-block j = i // 32, code i % 16): (j+1)*code - 0.5*j
    for i, want in ((0, 0.0), (17, 1.0), (31, 15.0), (40, 15.5), (63, 29.5), (64, -1.0),
                    (127, 58.5), (200, 53.0), (255, 116.5)):
        assert w[i] == want, (i, w[i], want)


def test_q4k_scale_packing_round_trip():
    """Every (scale, min) pair of every sub-block position survives ggml's
    packing and the repack's unpacking."""
    rng = np.random.default_rng(0)
    for trial in range(64):
        sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        if trial == 0:
            sc, mn = np.full(8, 63), np.full(8, 63)
        blk = known_block()
        blk[4:16] = ob.q4k_pack_scales(sc, mn)
        plane, sd, md, sq, mq = sa.q4k_repack(blk, 1, 256)
        assert (sq[0] == sc).all() and (mq[0] == 127 - mn).all(), (sc, mn, sq, mq)
        assert sd[0, 0] == blk[0:2].view(np.uint16)[0] and md[0, 0] == blk[2:4].view(np.uint16)[0]
        assert (plane[0] == blk[16:]).all()


@pytest.mark.parametrize("rows,cols,seed", [(3, 256, 1), (17, 2048, 2), (64, 4096, 3)])
def test_q4k_repack_equals_published_formula(rows, cols, seed):
    """Random blocks: the repacked FLAT record's dequantization (the SSF
    formula) equals dequantize_row_q4_K bit for bit, row by row."""
    blocks = ob.q4k_random_blocks(rows, cols, seed)
    v = ob.FlatView(*sa.q4k_repack(blocks, rows, cols), rows, cols)
    want = ob.q4k_dequant(blocks, rows, cols)
    for r in range(rows):
        np.testing.assert_array_equal(v.dequant(r), want[r], err_msg=f"row {r}")


def test_q4k_repack_refuses_partial_blocks():
    with pytest.raises(ValueError):
        sa.q4k_repack(np.zeros(144, np.uint8), 1, 128)


def known_q5_block(qh):
    """known_block's fields and nibbles with the given 32 qh bytes."""
    blk = np.zeros(176, np.uint8)
    k4 = known_block()
    blk[0:16] = k4[0:16]
    blk[16:48] = qh
    blk[48:] = k4[16:]
    return blk


def test_q5k_known_answers():
    """Values worked out by hand: code (i % 32) % 16 plus 16 where the fifth
    bit is set, weight (j+1)*code - 0.5*j for sub-block j = i // 32."""
    # every odd weight of every sub-block has its fifth bit
    w = ob.q5k_dequant(known_q5_block(np.where(np.arange(32) % 2 == 1, 0xFF, 0).astype(np.uint8)), 1, 256)[0]
    for i, want in ((0, 0.0), (17, 17.0), (31, 31.0), (40, 15.5), (63, 61.5), (64, -1.0),
                    (127, 122.5), (200, 53.0), (255, 244.5)):
        assert w[i] == want, (i, w[i], want)
    # qh[l] = 1 << (l % 8): weight l of sub-block j has it only where j == l % 8
    w = ob.q5k_dequant(known_q5_block((1 << (np.arange(32) % 8)).astype(np.uint8)), 1, 256)[0]
    for i, want in ((0, 16.0), (1, 1.0), (33, 33.5), (34, 3.5), (231, 180.5), (232, 60.5), (255, 244.5)):
        assert w[i] == want, (i, w[i], want)
    # no fifth bits, high nibbles 15 - (l % 16): odd sub-blocks read the high nibble
    blk = known_q5_block(np.zeros(32, np.uint8))
    l = np.arange(32) % 16
    blk[48:] = np.tile(l | ((15 - l) << 4), 4)
    w = ob.q5k_dequant(blk, 1, 256)[0]
    for i, want in ((0, 0.0), (32, 29.5), (47, -0.5), (64, -1.0), (96, 58.5), (255, -3.5)):
        assert w[i] == want, (i, w[i], want)


def test_q5k_repack_fields_and_bits():
    """Q4_K's fields and nibbles carry over unchanged; the 1-bit plane holds
    bit j of qh[l] as weight l of group j."""
    rng = np.random.default_rng(5)
    blk = known_q5_block(rng.integers(0, 256, 32, dtype=np.uint8))
    sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
    blk[4:16] = ob.q4k_pack_scales(sc, mn)
    (p4, p1), sd, md, sq, mq = sa.q5k_repack(blk, 1, 256)
    assert (sq[0] == sc).all() and (mq[0] == 127 - mn).all()
    assert sd[0, 0] == blk[0:2].view(np.uint16)[0] and md[0, 0] == blk[2:4].view(np.uint16)[0]
    assert (p4[0] == blk[48:]).all()
    bits = np.unpackbits(p1[0], bitorder="little").reshape(8, 32)
    want = (blk[16:48][None, :] >> np.arange(8)[:, None]) & 1
    assert (bits == want).all()


@pytest.mark.parametrize("rows,cols,seed", [(3, 256, 1), (17, 2048, 2), (64, 4096, 3)])
def test_q5k_repack_equals_published_formula(rows, cols, seed):
    """Random blocks: the repacked FLAT Q5 record's dequantization equals
    dequantize_row_q5_K bit for bit, row by row."""
    blocks = ob.q5k_random_blocks(rows, cols, seed)
    v = ob.FlatView(*sa.q5k_repack(blocks, rows, cols), rows, cols, nbits=5)
    want = ob.q5k_dequant(blocks, rows, cols)
    for r in range(rows):
        np.testing.assert_array_equal(v.dequant(r), want[r], err_msg=f"row {r}")


def test_q5k_repack_refuses_partial_blocks():
    with pytest.raises(ValueError):
        sa.q5k_repack(np.zeros(176, np.uint8), 1, 128)


KINDS = {
    "q4k": (ob.q4k_random_blocks, sa.q4k_repack, sa.Mat.from_q4k, ob.q4k_dequant, 4),
    "q5k": (ob.q5k_random_blocks, sa.q5k_repack, sa.Mat.from_q5k, ob.q5k_dequant, 5),
}


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["q4k", "q5k"])
@pytest.mark.parametrize("rows,cols,seed", [(4096, 4096, 11), (1000, 14336, 12)])
def test_kquant_on_the_gpu(kind, rows, cols, seed):
    """Uploaded as Q4_K or Q5_K: the unpacked codes are the blocks' codes
    (bit for bit); the GEMV and the SwiGLU GEMV on an int8 activation agree
    with the oracle's GEMV on the repacked record and with a
    double-precision product of the published dequantization (1e-3 of the
    largest output, rel-RMS 1e-4)."""
    gen, repack, upload, dequant, nbits = KINDS[kind]
    sa.init(0)
    blocks = gen(rows, cols, seed)
    m = upload(blocks, rows, cols)
    v = ob.FlatView(*repack(blocks, rows, cols), rows, cols, nbits=nbits)
    for r0 in (0, rows // 2, rows - 3):
        got = sa.unpack(m, r0, 3)
        for i in range(3):
            np.testing.assert_array_equal(got[i], v.codes(r0 + i), err_msg=f"codes row {r0 + i}")
    x = np.random.default_rng(seed).standard_normal(cols).astype(np.float32)
    q, s, u = ob.quantize_act(x)
    act = sa.Act(cols)
    xd = sa.DevBuf.of(x)
    sa.normq(xd, act)
    np.testing.assert_array_equal(act.read()[0], q)
    y = sa.DevBuf(rows * 4)
    sa.matvec(m, act, y)
    got = y.read(np.float32)
    want = v.matvec(q, s, u)
    xq = (q.astype(np.float64).reshape(-1, 32) * s.astype(np.float64)[:, None]).reshape(-1)
    brute = dequant(blocks, rows, cols).astype(np.float64) @ xq
    for ref, what in ((want, "oracle GEMV"), (brute, "published dequant x activation")):
        err = np.abs(got - ref)
        assert err.max() <= 1e-3 * np.abs(ref).max(), what
        assert np.sqrt((err ** 2).mean() / (ref ** 2).mean()) <= 1e-4, what
    up = upload(gen(rows, cols, seed + 100), rows, cols)
    h = sa.DevBuf(rows * 4)
    sa.matvec_swiglu(m, up, act, h)
    vu = ob.FlatView(*repack(gen(rows, cols, seed + 100), rows, cols), rows, cols, nbits=nbits)
    g, uu = want.copy(), vu.matvec(q, s, u)
    ob.oracle().orc_silu_mul(g.ctypes.data, uu.ctypes.data, rows)
    hg = h.read(np.float32)
    assert np.abs(hg - g).max() <= 1e-3 * np.abs(g).max()
    m.free()
    up.free()


# ------------------------------------------------- Q8_0, Q4_0, Q6_K: dequantized, then re-quantized
# These block types do not factor into the FLAT record's per-256 fp16 step
# times a per-32 integer, so they take the reference's own route for a GGUF:
# the float16 copy (transformers reading the file, tooling/sml_gguf.py:19-27)
# re-quantized by the quantizer (the GPU ingest, sml_hip_requant).

def f16(x):
    return np.array([x], np.float16).view(np.uint8)


def test_q8_0_known_answers():
    """d = 0.5: weight i of the block is 0.5 * code i; a second block with
    d = 3 (exact products); codes -128, -1, 0, 1, 127 included."""
    codes = np.array([-128, -1, 0, 1, 127] + list(range(-13, 14)), np.int8)
    b = np.concatenate([f16(0.5), codes.view(np.uint8), f16(3.0), codes[::-1].copy().view(np.uint8)])
    w = ob.gguf_dequant_f16(8, b, 1, 64)[0]
    assert w[0] == -64.0 and w[1] == -0.5 and w[2] == 0.0 and w[3] == 0.5 and w[4] == 63.5
    assert np.array_equal(w[:32], 0.5 * codes.astype(np.float32))
    assert w[32] == 3.0 * 13 and w[63] == -384.0


def test_q4_0_known_answers():
    """Byte j's low nibble is weight j, its high nibble weight j + 16; value
    d * (nibble - 8)."""
    qs = np.array([(j & 15) | ((15 - j) << 4) for j in range(16)], np.uint8)
    b = np.concatenate([f16(0.25), qs])
    w = ob.gguf_dequant_f16(2, b, 1, 32)[0]
    for j in range(16):
        assert w[j] == 0.25 * (j - 8), j
        assert w[j + 16] == 0.25 * (15 - j - 8), j


def q6k_block(code_at=None, d=1.0):
    """A Q6_K block with every code 32 (weight 0) except code_at = {weight:
    code}; scales[j] = j + 1. Bytes placed by hand from the layout: weight
    128h + 32k + l takes ql[64h + l + 32(k & 1)] (low nibble for k < 2, high
    for k >= 2) and bits 2k..2k+1 of qh[32h + l]."""
    ql = np.zeros(128, np.uint8)
    qh = np.full(64, 0xAA, np.uint8)          # code 32 = 0b10_0000: high pair 2 in every slot
    for wgt, c in (code_at or {}).items():
        h, i = divmod(wgt, 128)
        k, l = divmod(i, 32)
        bi = 64 * h + l + 32 * (k & 1)
        sh = 4 * (k >> 1)
        ql[bi] = (int(ql[bi]) & (0xFF ^ (15 << sh))) | ((c & 15) << sh)
        qi = 32 * h + l
        qh[qi] = (int(qh[qi]) & (0xFF ^ (3 << (2 * k)))) | ((c >> 4) << (2 * k))
    sc = np.arange(1, 17, dtype=np.int8)
    return np.concatenate([ql, qh, sc.view(np.uint8), f16(d)])


@pytest.mark.parametrize("wgt,code", [(0, 63), (37, 63), (70, 0), (101, 17), (127, 48), (128, 5), (200, 33),
                                      (255, 62)])
def test_q6k_known_answers(wgt, code):
    """One weight's code set: that weight is d * scales[w/16] * (code - 32)
    and every other weight 0 -- which pins the ql byte, the nibble, the qh
    bit pair and the scale each weight reads."""
    w = ob.gguf_dequant_f16(14, q6k_block({wgt: code}, d=0.5), 1, 256)[0]
    want = np.zeros(256, np.float32)
    want[wgt] = np.float32(0.5 * (wgt // 16 + 1) * (code - 32))
    assert np.array_equal(w, want), (wgt, np.flatnonzero(w), w[np.flatnonzero(w)])


def test_q6k_negative_scales_and_fp16_rounding():
    """Signed scales; products rounded once to fp16 (d = 0.1 is not exact:
    (d*sc)*q in float, then fp16)."""
    blk = q6k_block({i: (i * 7) % 64 for i in range(256)}, d=0.1)
    blk[192:208] = np.array([-128, -3, 5, 127, -1, 0, 2, 64, -64, 9, -9, 100, -100, 1, 33, -77], np.int8).view(np.uint8)
    w = ob.gguf_dequant_f16(14, blk, 1, 256)[0]
    d = np.float32(np.float16(0.1))
    sc = blk[192:208].view(np.int8).astype(np.float32)
    for i in (0, 17, 40, 95, 130, 255):
        v = (d * sc[i // 16]) * np.float32((i * 7) % 64 - 32)
        assert w[i] == np.float32(np.float16(v)), i


def _numpy_q6k(blocks):
    """gguf-py's published numpy formulation of Q6_K (reshapes and shifts
    over whole blocks), an independent statement of the same layout."""
    b = blocks.reshape(-1, 210)
    n = b.shape[0]
    ql, qh, sc, d = b[:, :128], b[:, 128:192], b[:, 192:208], b[:, 208:210]
    d = d.copy().view(np.float16).astype(np.float32)
    sc = sc.copy().view(np.int8).astype(np.float32)
    dd = (d * sc).reshape(n, 16, 1)
    lo = (ql.reshape(n, -1, 1, 64) >> np.array([0, 4], np.uint8).reshape(1, 1, 2, 1)) & np.uint8(15)
    lo = lo.reshape(n, -1, 32)
    hi = (qh.reshape(n, -1, 1, 32) >> np.array([0, 2, 4, 6], np.uint8).reshape(1, 1, 4, 1)) & np.uint8(3)
    hi = hi.reshape(n, -1, 32)
    q = (lo | (hi << np.uint8(4))).astype(np.int8) - np.int8(32)
    return (dd * q.reshape(n, 16, -1).astype(np.float32)).reshape(n, 256).astype(np.float16).astype(np.float32)


def test_q6k_equals_the_numpy_formulation():
    rng = np.random.default_rng(6)
    rows, cols = 7, 768
    blocks = rng.integers(0, 256, (rows, cols // 256, 210)).astype(np.uint8)
    blocks[..., 208:210] = (rng.standard_normal((rows, cols // 256)) * 0.01).astype(np.float16)[..., None].view(np.uint8)
    got = ob.gguf_dequant_f16(14, blocks, rows, cols)
    assert np.array_equal(got, _numpy_q6k(blocks).reshape(rows, cols))


def test_gguf_dequant_refuses_other_types_and_partial_blocks():
    with pytest.raises(ValueError):
        ob.gguf_dequant_f16(12, np.zeros(144, np.uint8), 1, 256)
    with pytest.raises(ValueError):
        ob.gguf_dequant_f16(14, np.zeros(210, np.uint8), 1, 128)
