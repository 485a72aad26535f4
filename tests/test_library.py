"""The C-ABI library: it loads, exports every symbol the public headers
declare, and fails cleanly (NULL / 0 with a reason, no exit) where it cannot
run -- as on a host without a GPU."""
import ctypes
import os
import re

import pytest

import sheep_amd as sa

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    names = set()
    for h in os.listdir(os.path.join(ROOT, "include")):
        src = open(os.path.join(ROOT, "include", h)).read()
        src = re.sub(r"//[^\n]*", "", src)
        for m in re.finditer(r"\b(sml_[a-z0-9_]+)\s*\(", src):
            names.add(m.group(1))
    return names


def test_exports_every_declared_symbol():
    lib = ctypes.CDLL(sa.LIB_PATH)
    names = declared()
    assert len(names) >= 30
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing


def test_reference_boundary_prototypes():
    src = open(os.path.join(ROOT, "include", "sml-gpu.h")).read()
    for proto in ["int sml_gpu_open(const char * path, int n_ctx, int threads, int gpu_layers, char * why, int nwhy);",
                  "const float * sml_gpu_prefill(const int * ids, int pos0, int n);",
                  "const float * sml_gpu_step(int tok, int pos);",
                  "int sml_gpu_layers(int * of);",
                  "void sml_gpu_prompt_mode(int level);",
                  "int sml_gpu_decode_cpu(int on);",
                  "void sml_gpu_set_middle(int layers, int (*fn)(float * rows, int pos0, int n));"]:
        assert proto in src, proto


def _has_gpu():
    return os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK | os.W_OK)


@pytest.mark.skipif(_has_gpu(), reason="checks the no-GPU failure path")
def test_open_without_gpu_fails_with_reason(tmpdir_s):
    p = tmpdir_s / "nogpu.ssf"
    sa.synth_model(p, n_layer=1, n_embd=256, n_head=2, n_head_kv=1, n_ff=512, n_vocab=300, seed=1)
    why = ctypes.create_string_buffer(512)
    assert sa.lib().sml_gpu_open(str(p).encode(), 64, 1, 0, why, 512) == 0
    assert why.value
    assert not sa.lib().sml_gpu_step(1, 0)
    assert not sa.lib().sml_gpu_prefill((ctypes.c_int * 2)(1, 2), 0, 2)
    of = ctypes.c_int(-1)
    assert sa.lib().sml_gpu_layers(ctypes.byref(of)) == 0 and of.value == 0
    assert sa.lib().sml_gpu_generate(1, 0, 4, (ctypes.c_int * 4)()) == -1


def test_refuses_unsupported_file_before_touching_the_gpu(tmpdir_s):
    p = tmpdir_s / "bad.ssf"
    p.write_bytes(b"NOPE" + bytes(5000))
    why = ctypes.create_string_buffer(512)
    assert sa.lib().sml_gpu_open(str(p).encode(), 64, 1, 0, why, 512) == 0
    assert b"not an SSF file" in why.value


def test_kernel_abi_reports_errors_without_gpu():
    if _has_gpu():
        pytest.skip("no-GPU path")
    assert not sa.lib().sml_hip_malloc(16)
    assert sa.lib().sml_hip_last_error()
