"""SSF format: struct layout, the seeded writer, and loader acceptance rules.

The layout is pinned against the reference's own packed structs (compiled
from its sml-model.h) and the acceptance rules against the reference loader
sml_model_open (sml/sml-model.c:26-72,173-260): every mutation below must be
accepted or refused by both the same way.
"""
import ctypes
import hashlib
import os
import shutil
import struct

import numpy as np
import pytest

import sheep_amd as sa
from oracle import bind as ob
from sheep_amd.ssf import HEADER_SIZE, REC_SIZE, SSF

needs_ref = pytest.mark.skipif(not ob.have_ref(), reason="reference CPU build not present")


def test_struct_sizes_match_reference_build():
    if not ob.have_ref():
        assert (HEADER_SIZE, REC_SIZE) == (228, 248)
        return
    lay = (ctypes.c_long * 12)()
    ob.ref().ref_layout(lay)
    assert lay[0] == HEADER_SIZE and lay[1] == REC_SIZE
    # table_off, flags, n_expert_used, moe_flags, gdn_dk / perm_off, mq_n, codes_off, nbits, rope_theta
    assert list(lay[2:12]) == [76, 152, 168, 172, 224, 128, 168, 176, 244, 36]


def test_synthetic_file_is_deterministic(tmpdir_s):
    a, b = tmpdir_s / "d1.ssf", tmpdir_s / "d2.ssf"
    for p in (a, b):
        sa.synth_model(p, n_layer=1, n_embd=256, n_head=2, n_head_kv=1, n_ff=512, n_vocab=300, seed=11,
                       random_perm=True)
    assert hashlib.sha256(a.read_bytes()).digest() == hashlib.sha256(b.read_bytes()).digest()


@pytest.mark.parametrize("nb", range(2, 9))
def test_writer_fields_and_codes(tmpdir_s, nb):
    p = tmpdir_s / f"wf{nb}.ssf"
    sa.synth_matrix(p, 8, 512, nbits=nb, random_perm=True, seed=nb)
    t = SSF(p)["w"]
    assert t.nbits == nb and t.rows == 8 and t.cols == 512
    sq = t.sq.reshape(8, 16)
    mq = t.mq.reshape(8, 16)
    assert sq.min() >= 1 and mq.max() <= 254
    perm = t.perm
    assert sorted(perm.tolist()) == list(range(512))
    codes = np.stack([ob.unpack(t, r) for r in range(8)])
    assert codes.max() <= (1 << nb) - 1
    # codes are uniform over the width's range: every value appears
    assert len(np.unique(codes)) == 1 << nb


@needs_ref
def test_reference_loader_accepts_synthetic_decoder(tmpdir_s):
    p = tmpdir_s / "acc.ssf"
    sa.synth_model(p, n_layer=2, n_embd=256, n_head=2, n_head_kv=1, n_ff=512, n_vocab=300, qkv_bias=True, seed=3)
    m = ob.RefModel(p, 16, threads=1)
    lg = m.forward(1, 0)
    assert lg.shape == (300,) and np.isfinite(lg).all()
    m.close()


def _mutations():
    # (name, header field offset or record-relative offset, struct fmt, value, target)
    H, R = "hdr", "rec"
    return [
        ("bad magic", H, 0, "4s", b"GGUF"),
        ("newer version", H, 4, "I", 10),
        ("zero levels", H, 48, "I", 0),
        ("five levels", H, 48, "I", 5),
        ("unknown flag", H, 152, "I", 1 << 7),
        ("minneg without scale6", H, 152, "I", 4),
        ("table past end", H, 76, "Q", 1 << 40),
        ("group 64", H, 44, "I", 64),
        ("zero rows", R, 68, "I", 0),
        ("unknown kind", R, 64, "I", 7),
        ("flat width 1", R, 244, "I", 1),
        ("flat width 9", R, 244, "I", 9),
        ("codes past end", R, 176, "Q", 1 << 40),
        ("sd past end", R, 96, "Q", 1 << 40),
        ("perm inside header", R, 128, "Q", 16),
        ("layout 2", R, 240, "I", 2),
    ]


@needs_ref
@pytest.mark.parametrize("case", _mutations(), ids=lambda c: c[0])
def test_loader_rejections_match_reference(tmpdir_s, case):
    name, where, off, fmt, val = case
    src = tmpdir_s / "base.ssf"
    if not src.exists():
        sa.synth_matrix(src, 8, 256, nbits=4, seed=1)
    p = tmpdir_s / ("mut_" + name.replace(" ", "_") + ".ssf")
    shutil.copy(src, p)
    hdr = SSF(src).hdr
    base = 0 if where == "hdr" else hdr["table_off"]
    with open(p, "r+b") as f:
        f.seek(base + off)
        f.write(struct.pack("<" + fmt, val))
    why = ctypes.create_string_buffer(512)
    mine = sa.lib().ssf_open  # exported reader
    mine.restype = ctypes.c_int
    mine.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int]
    fbuf = ctypes.create_string_buffer(64)
    ok_mine = mine(fbuf, str(p).encode(), why, 512)
    if ok_mine:
        close = sa.lib().ssf_close
        close.argtypes = [ctypes.c_void_p]
        close(fbuf)
    h = ob.ref().ref_open(str(p).encode(), 0, 1, 0)
    ok_ref = bool(h)
    if h:
        ob.ref().ref_close(h)
    assert ok_mine == ok_ref, f"{name}: mine {ok_mine}, reference {ok_ref} ({why.value.decode()})"
    assert not ok_ref, name
    assert why.value, "a refusal carries a reason"


def test_server_vocab_section(tmp_path):
    """The byte-fallback vocabulary the server test appends lands where the
    header's tok_off / tok_n say, in the reference's layout
    (sml/sml-vocab.c:64-78: n_tokens, n_merges, bos, eos, offsets, bytes),
    and the tensors still read the same."""
    from test_gpu_server import SPECIALS, add_vocab
    p = tmp_path / "v.ssf"
    sa.synth_model(p, n_layer=1, n_embd=256, n_head=2, n_head_kv=1, n_ff=512, n_vocab=600, seed=3)
    before = np.array(SSF(p)["token_embd.weight"].plane(0)[:4096])
    add_vocab(str(p), 600)
    f = SSF(p)
    off, n = f.hdr["tok_off"], f.hdr["tok_n"]
    assert off % 256 == 0 and off + n == os.path.getsize(p)
    blob = bytes(f.mm[off:off + n])
    nt, nm, bos, eos = struct.unpack_from("<4I", blob, 0)
    assert (nt, nm, bos, eos) == (600, 0, 256, 258)
    offs = struct.unpack_from(f"<{nt + 1}I", blob, 16)
    data = blob[16 + 4 * (nt + 1):]
    tok = lambda i: data[offs[i]:offs[i + 1]]
    assert tok(0) == b"<0x00>" and tok(255) == b"<0xFF>"
    assert [tok(256 + i).decode() for i in range(3)] == SPECIALS
    assert tok(599) == "▁w599".encode() and offs[-1] == len(data)
    np.testing.assert_array_equal(np.array(f["token_embd.weight"].plane(0)[:4096]), before)
