"""Write the golden vectors under tests/golden/ from the reference engine's own
CPU path (oracle/_ref/libsmlref.so, compiled from the reference's C sources).

The reference ships no data fixtures, so these are produced here: seeded
inputs (the synthetic SSF files are regenerated from their seeds and checked
by sha256) and the reference's outputs on them. Run from the repository root:

    python tests/golden/make_golden.py
"""
import hashlib
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import sheep_amd as sa  # noqa: E402
from oracle import bind as ob  # noqa: E402
from sheep_amd.ssf import SSF  # noqa: E402

OUT = os.path.join(ROOT, "tests", "golden")


def sha(path):
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


def act_vectors():
    rng = np.random.default_rng(2024)
    xs = [rng.standard_normal(1024).astype(np.float32)]
    # edge cases: an all-zero group, exact half-way products, a huge outlier, denormals
    e = rng.standard_normal(1024).astype(np.float32)
    e[0:32] = 0.0
    e[32:64] = np.arange(32, dtype=np.float32) * 0.5 - 8.0
    e[64] = 1e30
    e[96:128] = np.float32(1e-40)
    xs.append(e)
    out = {}
    for i, x in enumerate(xs):
        for per256 in (0, 1):
            q, s, u = ob.ref_quantize_act(x, per256=bool(per256))
            out[f"x{i}"] = x
            out[f"q{i}_{per256}"], out[f"s{i}_{per256}"], out[f"u{i}_{per256}"] = q, s, u
    np.savez_compressed(os.path.join(OUT, "act_quant.npz"), **out)


def width_vectors(tmp):
    out = {}
    for nb in range(2, 9):
        p = os.path.join(tmp, f"w{nb}.ssf")
        sa.synth_matrix(p, 16, 256, nbits=nb, random_perm=True, seed=100 + nb)
        t = SSF(p)["w"]
        x = np.random.default_rng(nb).standard_normal(256).astype(np.float32)
        q, s, u = ob.ref_quantize_act(x)
        out[f"sha{nb}"] = np.frombuffer(bytes.fromhex(sha(p)), np.uint8)
        out[f"x{nb}"] = x
        out[f"y{nb}"] = ob.ref_matvec(t, q, s, u)
        out[f"deq{nb}"] = np.stack([ob.ref_dequant_row(t, r) for r in range(16)])
    np.savez_compressed(os.path.join(OUT, "widths.npz"), **out)


def decoder_vectors(tmp):
    p = os.path.join(tmp, "tiny.ssf")
    sa.synth_model(p, n_layer=2, n_embd=256, n_head=2, n_head_kv=1, n_ff=512, n_vocab=1000,
                   qkv_bias=True, random_perm=True, seed=7)
    m = ob.RefModel(p, 32, threads=1)
    toks, logits = [5], []
    for pos in range(16):
        lg = m.forward(toks[-1], pos)
        logits.append(lg)
        toks.append(int(np.argmax(lg)))
    m.close()
    route = {}
    rng = np.random.default_rng(9)
    lgs = rng.standard_normal((64, 8)).astype(np.float32)
    lgs[0] = 0.5                      # all tied
    lgs[1, 3] = lgs[1, 5] = 2.0       # a tie for first
    sel = np.zeros((64, 2), np.int32)
    w = np.zeros((64, 2), np.float32)
    for i in range(64):
        ob.ref().ref_moe_route(lgs[i].ctypes.data, 8, 2, 1, sel[i].ctypes.data, w[i].ctypes.data)
    np.savez_compressed(os.path.join(OUT, "decoder.npz"), sha=np.frombuffer(bytes.fromhex(sha(p)), np.uint8),
                        tokens=np.array(toks, np.int32), logits=np.stack(logits), route_lg=lgs,
                        route_sel=sel, route_w=w)


if __name__ == "__main__":
    if not ob.have_ref():
        sys.exit("oracle/_ref/libsmlref.so is not built: run make -C oracle where the reference is present")
    with tempfile.TemporaryDirectory() as tmp:
        act_vectors()
        width_vectors(tmp)
        decoder_vectors(tmp)
    print("golden vectors written to", OUT)
