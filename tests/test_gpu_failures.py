"""The boundary's failure contract (sml/sml-gpu.h, sml/sml-gpu-fwd.c:23-27):
no entry point ends the process; a failed call returns NULL or 0, and the
library keeps working afterwards.

Failures are made on the host, never on the device: sml_hip_fail_after(n)
turns the n-th HIP call the library makes from then on into an error, as a
real device error would arrive, at every point of sml_gpu_open (uploads,
graph capture), of a prompt and of a step. Under the reference's own server
(oracle/_ref/sml-server), SML_GPU_FAIL makes one entry point fail: the server
must retire the GPU and finish the reply on its CPU path
(sml/sml-server.c:204-265).
"""
import os

import numpy as np
import pytest

import sheep_amd as sa

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    p = tmp_path_factory.mktemp("fail") / "m.ssf"
    sa.synth_model(p, n_layer=2, n_embd=512, n_head=4, n_head_kv=2, n_ff=1024, n_vocab=2000,
                   qkv_bias=True, random_perm=True, seed=31)
    return p


IDS = np.random.default_rng(4).integers(0, 2000, 24).astype(np.int32)


def clean_run(path, exact=False):
    """Prompt of 20 ids (batched), then 4 steps: the logits of each."""
    d = sa.Decoder(path, n_ctx=64, exact=exact)
    try:
        out = [d.prefill(IDS[:20], 0, 2000)]
        out += [d.step(int(IDS[20 + i]), 20 + i, 2000) for i in range(4)]
    finally:
        d.close()
    return out


def calls_of(fn):
    before = sa.lib().sml_hip_call_count()
    fn()
    return sa.lib().sml_hip_call_count() - before


@pytest.mark.parametrize("exact", [False, True])
def test_open_fails_cleanly_at_every_point(model, exact):
    """Every k-th HIP call of sml_gpu_open failing (allocation, upload, code
    lookup, graph capture): open returns 0 with a reason, and the next open
    decodes exactly as a clean one."""
    want = clean_run(model, exact)
    n = calls_of(lambda: sa.Decoder(model, n_ctx=64, exact=exact).close())
    assert n > 50
    why = sa.ctypes.create_string_buffer(512)
    points = sorted(set(list(range(0, 40)) + list(range(40, n, max(1, n // 60))) + [n - 1]))
    for k in points:
        sa.lib().sml_hip_fail_after(k)
        os.environ["SML_EXACT"] = "1" if exact else "0"
        try:
            ok = sa.lib().sml_gpu_open(str(model).encode(), 64, 1, 0, why, 512)
        finally:
            sa.lib().sml_hip_fail_after(-1)
            del os.environ["SML_EXACT"]
        assert ok == 0, f"open survived a failure at HIP call {k} of {n}"
        assert why.value, k
        assert not sa.lib().sml_gpu_step(1, 0)
    got = clean_run(model, exact)
    for a, b in zip(got, want):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("level", [0, 1])
def test_prompt_and_step_fail_then_retry(model, level):
    """A failure at any HIP call of a prompt or a step: the call returns NULL;
    the same call again (same ids, same positions) then gives the clean
    run's logits, and decoding continues as if nothing had failed."""
    want = clean_run(model)
    d = sa.Decoder(model, n_ctx=64)
    try:
        d.prompt_mode(level)
        d.prefill(IDS[:20], 0, 2000)            # the first batched prompt also allocates its buffers
        n_pre = calls_of(lambda: d.prefill(IDS[:20], 0, 2000))
        n_step = calls_of(lambda: d.step(int(IDS[20]), 20, 2000))
        for k in sorted(set([0, 1, 2, n_pre // 2, n_pre - 1])):
            sa.lib().sml_hip_fail_after(k)
            p = sa.lib().sml_gpu_prefill(IDS[:20].ctypes.data_as(sa.P(sa.c_int)), 0, 20)
            sa.lib().sml_hip_fail_after(-1)
            assert not p, f"prefill survived a failure at HIP call {k} of {n_pre}"
            np.testing.assert_array_equal(d.prefill(IDS[:20], 0, 2000), want[0])
        for k in range(n_step):
            sa.lib().sml_hip_fail_after(k)
            p = sa.lib().sml_gpu_step(int(IDS[20]), 20)
            sa.lib().sml_hip_fail_after(-1)
            assert not p, f"step survived a failure at HIP call {k} of {n_step}"
        for i in range(4):
            np.testing.assert_array_equal(d.step(int(IDS[20 + i]), 20 + i, 2000), want[1 + i])
    finally:
        d.close()


def test_generate_fails_then_recovers(model):
    d = sa.Decoder(model, n_ctx=64)
    try:
        want = list(d.generate(5, 0, 12))
        n = calls_of(lambda: d.generate(5, 0, 12))
        out = (sa.ctypes.c_int * 12)()
        for k in (0, n // 2, n - 1):
            sa.lib().sml_hip_fail_after(k)
            rc = sa.lib().sml_gpu_generate(5, 0, 12, out)
            sa.lib().sml_hip_fail_after(-1)
            assert rc == -1
            assert list(d.generate(5, 0, 12)) == want
    finally:
        d.close()


def test_kernel_level_calls_fail_cleanly():
    """The kernel-level ABI (include/sml-hip.h) returns -1 / NULL with a
    reason, and the next call works."""
    sa.init(0)
    sa.lib().sml_hip_fail_after(0)
    p = sa.lib().sml_hip_malloc(1024)
    sa.lib().sml_hip_fail_after(-1)
    assert not p and sa.lib().sml_hip_last_error()
    b = sa.DevBuf.of(np.arange(16, dtype=np.float32))
    sa.lib().sml_hip_fail_after(0)
    assert sa.lib().sml_hip_memset(b.ptr, 0, 64) == -1
    sa.lib().sml_hip_fail_after(-1)
    assert sa.lib().sml_hip_h2d(b.ptr, np.full(16, 7, np.float32).ctypes.data, 64) == 0
    np.testing.assert_array_equal(b.read(np.float32), np.full(16, 7, np.float32))
