"""A layer split on the GPU: sml_gpu_open's gpu_layers below the layer count.

The reference keeps that many leading layers on its card and finishes the
rest on its CPU engine (sml/sml-gpu-fwd.c:2028-2097, 1571-1590, 1745-1756).
Here the leading layers keep their matrices in HBM and the others are
streamed: their matrices sit in pinned host memory and cross to one staging
region in HBM ahead of each use, and the same kernels run on the same bytes.
So every path of a split model gives the whole model's logits bit for bit:
stepping, the three prompt levels, exact mode and the batched step.

A split model reads a prompt layer by layer (each streamed layer crosses the
host link once per prompt), every chunk computing what it computes in the
whole model's chunk-by-chunk order.

A middle stage (sml_gpu_set_middle, sml/sml-gpu.h:30-34) receives the hidden
rows after the layers on the card and runs the next layers itself. Checked
on a file whose middle layer adds nothing (its o and down steps are zero), so
an identity stage must give the whole model's logits, and with the positions
and row counts the reference's stage receives.
"""
import ctypes
import os
import shutil

import numpy as np
import pytest

import sheep_amd as sa
from sheep_amd.ssf import SSF

pytestmark = pytest.mark.gpu

V = 1000
SHAPE = dict(n_layer=6, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=V)
IDS = (np.arange(40, dtype=np.int32) * 37 + 11) % V


@pytest.fixture(scope="module", autouse=True)
def device():
    sa.init(0)


def same_bits(got, want, what):
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, (f"{what}: {bad.size} of {got.size} differ, first at {bad[0]}: "
                           f"{got[bad[0]]!r} vs {want[bad[0]]!r}")


def model(tmpdir_s, name, **kw):
    p = tmpdir_s / f"split_{name}.ssf"
    if not p.exists():
        sa.synth_model(p, n_ctx_train=256, **{**SHAPE, **kw})
    return p


def run(path, gpu_layers, exact=False):
    """Logits of: a 40-id prompt at levels 0, 1 and 2 (level 2 skipped in
    exact mode), each followed by 3 greedy steps."""
    dec = sa.Decoder(path, n_ctx=256, gpu_layers=gpu_layers, exact=exact)
    out = []
    try:
        for level in ([0, 1] if exact else [0, 1, 2]):
            dec.prompt_mode(level)
            lg = dec.prefill(IDS, 0, V)
            out.append(lg)
            for i in range(3):
                lg = dec.step(int(np.argmax(lg)), len(IDS) + i, V)
                out.append(lg)
        return out, (dec.gpu_layers, dec.n_layer)
    finally:
        dec.close()


@pytest.mark.parametrize("kind", ["q4", "q6_perm_bias"])
def test_split_equals_whole_model(tmpdir_s, kind):
    kw = dict(nbits=4) if kind == "q4" else dict(nbits=6, random_perm=True, qkv_bias=True, tied=True)
    p = model(tmpdir_s, kind, **kw)
    whole, counts = run(p, 0)
    assert counts == (6, 6)
    for k in (1, 4):
        got, counts = run(p, k)
        assert counts == (k, 6), counts
        for i, (g, w) in enumerate(zip(got, whole)):
            same_bits(g, w, f"{kind}, {k} of 6 layers on the card, call {i}")


def test_split_exact_mode_equals_whole_model(tmpdir_s):
    p = model(tmpdir_s, "q4")
    whole, _ = run(p, 0, exact=True)
    got, counts = run(p, 2, exact=True)
    assert counts == (2, 6)
    for i, (g, w) in enumerate(zip(got, whole)):
        same_bits(g, w, f"exact mode, 2 of 6 layers on the card, call {i}")


def batched(path, gpu_layers, ns=5):
    dec = sa.Decoder(path, n_ctx=256, gpu_layers=gpu_layers)
    try:
        dec.slots(ns)
        for b in range(ns):
            dec.prefill_slot(b, IDS[: 10 + 3 * b], 0, V)
        out = []
        for i in range(3):
            out.append(dec.step_multi([(7 * b + i) % V for b in range(ns)], [10 + 3 * b + i for b in range(ns)],
                                      list(range(ns)), V))
        return out
    finally:
        dec.close()


def test_split_batched_step_equals_whole_model(tmpdir_s):
    """Five slots (the per-256 regime) and their batched prompts."""
    p = model(tmpdir_s, "q4")
    whole = batched(p, 0)
    got = batched(p, 3)
    for i, (g, w) in enumerate(zip(got, whole)):
        same_bits(g, w, f"batched step {i}, 3 of 6 layers on the card")


def test_split_layer_counts(tmpdir_s, monkeypatch):
    p = model(tmpdir_s, "q4")
    for want, arg in ((6, 6), (6, 99), (5, 5)):
        dec = sa.Decoder(p, n_ctx=256, gpu_layers=arg)
        try:
            assert (dec.gpu_layers, dec.n_layer) == (want, 6)
        finally:
            dec.close()
    monkeypatch.setenv("SML_GPU_LAYERS", "2")
    dec = sa.Decoder(p, n_ctx=256, gpu_layers=0)
    try:
        assert (dec.gpu_layers, dec.n_layer) == (2, 6)
    finally:
        dec.close()
    # left to the free memory: a reserve larger than any card leaves room for
    # no layer, so the open keeps the first one (the reference's least)
    monkeypatch.delenv("SML_GPU_LAYERS")
    monkeypatch.setenv("SML_SPLIT_RESERVE_MB", "10000000")
    got, counts = run(p, 0)
    assert counts == (1, 6), counts
    monkeypatch.delenv("SML_SPLIT_RESERVE_MB")
    whole, _ = run(p, 0)
    for i, (g, w) in enumerate(zip(got, whole)):
        same_bits(g, w, f"split chosen by the free memory, call {i}")


def test_split_refuses_a_mixture_of_experts_model(tmpdir_s):
    p = tmpdir_s / "split_moe.ssf"
    if not p.exists():
        sa.synth_model(p, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=256, n_vocab=V, n_ctx_train=256,
                       n_expert=4, n_expert_used=2)
    with pytest.raises(sa.HipError, match="mixture-of-experts"):
        sa.Decoder(p, n_ctx=256, gpu_layers=1)


MIDDLE = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.POINTER(ctypes.c_float), ctypes.c_int, ctypes.c_int)


def quiet_layer_model(tmpdir_s, layer=3):
    """The q4 file with layer `layer`'s o and down steps (sd) and min steps
    (md) zeroed: the layer adds nothing to the residual stream."""
    src = model(tmpdir_s, "q4")
    p = tmpdir_s / f"split_quiet{layer}.ssf"
    if not p.exists():
        shutil.copy(src, p)
        recs = SSF(src).tensors
        mm = np.memmap(p, dtype=np.uint8, mode="r+")
        for nm in (f"blk.{layer}.attn_output.weight", f"blk.{layer}.ffn_down.weight"):
            r = recs[nm].rec
            mm[r["sd_off"]:r["sd_off"] + r["sd_bytes"]] = 0
            if r["md_bytes"]:
                mm[r["md_off"]:r["md_off"] + r["md_bytes"]] = 0
        mm.flush()
        del mm
    return p


def test_middle_stage(tmpdir_s):
    p = quiet_layer_model(tmpdir_s)
    whole, _ = run(p, 0)
    calls = []

    def identity(rows, pos0, n):
        x = np.ctypeslib.as_array(rows, shape=(n, SHAPE["n_embd"]))
        calls.append((pos0, n, bool(np.isfinite(x).all() and np.abs(x).max() > 0)))
        return 1

    cb = MIDDLE(identity)
    sa.lib().sml_gpu_set_middle(1, ctypes.cast(cb, ctypes.c_void_p))
    try:
        got, counts = run(p, 3)
        assert counts == (3, 6)
        for i, (g, w) in enumerate(zip(got, whole)):
            same_bits(g, w, f"identity middle stage for the quiet layer, call {i}")
        steps = [(40, 1, True), (41, 1, True), (42, 1, True)]
        # level 0 a token at a time; levels 1 and 2 read a split model's
        # prompt layer by layer, so the stage gets every row at once
        want = ([(i, 1, True) for i in range(40)] + steps
                + [(0, 40, True)] + steps
                + [(0, 40, True)] + steps)
        assert calls == want, calls
        # a stage that fails fails the call
        dec = sa.Decoder(p, n_ctx=256, gpu_layers=3)
        try:
            fail = MIDDLE(lambda rows, pos0, n: 0)
            sa.lib().sml_gpu_set_middle(1, ctypes.cast(fail, ctypes.c_void_p))
            with pytest.raises(sa.HipError):
                dec.prefill(IDS, 0, V)
            # the batched step serves several sequences: refused with a stage set
            sa.lib().sml_gpu_set_middle(1, ctypes.cast(cb, ctypes.c_void_p))
            dec.slots(2)
            with pytest.raises(sa.HipError, match="middle stage"):
                dec.step_multi([1, 2], [0, 0], [0, 1], V)
        finally:
            dec.close()
    finally:
        sa.lib().sml_gpu_set_middle(0, None)
