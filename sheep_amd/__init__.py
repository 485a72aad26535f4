"""MI355X-native SML decode path: ctypes bindings over libsmlhip.so.

The library (built from sheep_amd/csrc by __graft_entry__.build()) carries the
C host and the gfx950 code object. Nothing here computes on the CPU in place of
the GPU: if the library is missing, every entry point raises.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# SML_HIP_LIB points at another build of the same library (tuning experiments)
LIB_PATH = os.environ.get("SML_HIP_LIB") or os.path.join(HERE, "libsmlhip.so")

_lib = None

c_int, c_float, c_size_t, c_char_p, c_void_p = ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_char_p, ctypes.c_void_p
c_long, c_uint64 = ctypes.c_long, ctypes.c_uint64
P = ctypes.POINTER


class SynthSpec(ctypes.Structure):
    """ssf_synth_spec (sheep_amd/csrc/ssf.h)."""
    _fields_ = [("n_layer", ctypes.c_uint32), ("n_embd", ctypes.c_uint32), ("n_head", ctypes.c_uint32),
                ("n_head_kv", ctypes.c_uint32), ("n_ff", ctypes.c_uint32), ("n_vocab", ctypes.c_uint32),
                ("n_ctx_train", ctypes.c_uint32), ("rope_theta", c_float), ("rms_eps", c_float),
                ("nbits", c_int), ("tied", c_int), ("qkv_bias", c_int), ("random_perm", c_int),
                ("n_expert", c_int), ("n_expert_used", c_int), ("moe_flags", ctypes.c_uint32),
                ("step_sigma", c_float), ("router_sigma", c_float), ("seed", c_uint64), ("zero_mean", c_int),
                ("moe_scale", c_float), ("moe_groups", ctypes.c_uint32), ("moe_topk_group", ctypes.c_uint32),
                ("exp_bias", c_int), ("n_ff_shexp", c_int), ("shexp_gate", c_int)]


# (name, restype, argtypes) of every export
_SIGS = [
    ("sml_gpu_open", c_int, [c_char_p, c_int, c_int, c_int, c_char_p, c_int]),
    ("sml_gpu_prefill", P(c_float), [P(c_int), c_int, c_int]),
    ("sml_gpu_step", P(c_float), [c_int, c_int]),
    ("sml_gpu_layers", c_int, [P(c_int)]),
    ("sml_gpu_prompt_mode", None, [c_int]),
    ("sml_gpu_decode_cpu", c_int, [c_int]),
    ("sml_gpu_set_middle", None, [c_int, c_void_p]),
    ("sml_gpu_close", None, []),
    ("sml_gpu_generate", c_int, [c_int, c_int, c_int, P(c_int)]),
    ("sml_gpu_last_ms", c_float, []),
    ("sml_gpu_weight_bytes", c_uint64, []),
    ("sml_gpu_last_error", c_char_p, []),
    ("sml_gpu_slots", c_int, [c_int]),
    ("sml_gpu_prefill_slot", P(c_float), [c_int, P(c_int), c_int, c_int]),
    ("sml_gpu_step_multi", c_int, [P(c_int), P(c_int), P(c_int), c_int, c_void_p]),
    ("sml_gpu_exact", c_int, []),
    ("sml_hip_init", c_int, [c_int, c_char_p, c_int]),
    ("sml_hip_last_error", c_char_p, []),
    ("sml_hip_malloc", c_void_p, [c_size_t]),
    ("sml_hip_free", c_int, [c_void_p]),
    ("sml_hip_h2d", c_int, [c_void_p, c_void_p, c_size_t]),
    ("sml_hip_d2h", c_int, [c_void_p, c_void_p, c_size_t]),
    ("sml_hip_memset", c_int, [c_void_p, c_int, c_size_t]),
    ("sml_hip_sync", c_int, []),
    ("sml_hip_fail_after", None, [c_long]),
    ("sml_hip_set_exact", None, [c_int]),
    ("sml_hip_call_count", c_long, []),
    ("sml_hip_mat_upload", c_void_p, [P(c_void_p), c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int]),
    ("sml_hip_mat_from_file", c_void_p, [c_char_p, c_char_p]),
    ("sml_hip_mat_from_q4k", c_void_p, [c_void_p, c_int, c_int]),
    ("sml_hip_q4k_repack", c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("sml_hip_mat_from_q5k", c_void_p, [c_void_p, c_int, c_int]),
    ("sml_hip_q5k_repack", c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                   c_void_p]),
    ("sml_hip_mat_free", None, [c_void_p]),
    ("sml_hip_mat_info", c_int, [c_void_p, P(c_int), P(c_int), P(c_int)]),
    ("sml_hip_mat_bytes", c_size_t, [c_void_p]),
    ("sml_hip_normq", c_int, [c_void_p, c_void_p, c_void_p, c_float, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int]),
    ("sml_hip_matvec", c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("sml_hip_matvec_swiglu", c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("sml_hip_matvec_normq", c_int, [c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_void_p]),
    ("sml_hip_matvec_swiglu_fused", c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_void_p,
                                            c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("sml_hip_time_matvec", c_int, [P(c_void_p), c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, P(c_float)]),
    ("sml_hip_gemv_timeline", c_int, [P(c_void_p), c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p,
                                      c_int]),
    ("sml_hip_unpack", c_int, [c_void_p, c_int, c_int, c_void_p]),
    ("sml_hip_time_read", c_int, [P(c_void_p), c_int, c_size_t, c_int, c_int, P(c_float)]),
    ("sml_hip_copy", c_int, [c_void_p, c_void_p, c_size_t]),
    ("sml_hip_gemm", c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    ("sml_hip_gemm_swiglu", c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    ("sml_hip_gemm_sb", c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    ("sml_hip_gemm_swiglu_sb", c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    ("sml_hip_moe_regime", c_int, [c_void_p, c_int]),
    ("sml_hip_moe_from_file", c_void_p, [c_char_p, c_int, c_int]),
    ("sml_hip_moe_free", None, [c_void_p]),
    ("sml_hip_moe_info", c_int, [c_void_p, P(c_int), P(c_int), P(c_int), P(c_size_t)]),
    ("sml_hip_moe_ffn", c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("sml_hip_moe_time", c_int, [c_void_p, c_void_p, c_int, c_void_p, c_int, P(c_float), c_void_p]),
    ("sml_hip_gptq_upload", c_void_p, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int]),
    ("sml_hip_gptq_upload_gidx", c_void_p, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int]),
    ("sml_hip_awq_upload", c_void_p, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int]),
    ("sml_hip_gptq_free", None, [c_void_p]),
    ("sml_hip_gptq_bytes", c_size_t, [c_void_p]),
    ("sml_hip_gptq_matvec", c_int, [c_void_p, c_void_p, c_void_p]),
    ("sml_hip_gptq_unpack", c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p]),
    ("sml_hip_gptq_time", c_int, [P(c_void_p), c_int, c_void_p, c_void_p, c_int, P(c_float)]),
    ("sml_hip_embed", c_int, [c_void_p, c_void_p, c_void_p, c_void_p]),
    ("sml_hip_attn_part_floats", c_size_t, [c_int, c_int, c_int]),
    ("sml_hip_attention", c_int, [c_void_p] * 8 + [c_int] * 4 + [c_void_p, c_void_p]),
    ("sml_hip_attention_q", c_int, [c_void_p] * 8 + [c_int] * 4 + [c_void_p] * 5),
    ("sml_hip_attention_prompt", c_int, [c_void_p, c_int, c_int] + [c_void_p] * 4 + [c_int] * 4 + [c_void_p] * 2),
    ("sml_hip_softmax_sum", c_int, [c_void_p, c_int, c_void_p]),
    ("sml_hip_argmax", c_int, [c_void_p, c_int, c_void_p]),
    ("sml_hip_argmax_noalloc", c_int, [c_void_p, c_int, c_void_p]),
    ("ssf_synth_model", c_int, [c_char_p, P(SynthSpec), c_char_p, c_int]),
    ("ssf_synth_matrix", c_int, [c_char_p, c_int, c_int, c_int, c_int, c_float, c_uint64, c_char_p, c_int]),
    ("ssf_f32_to_f16", ctypes.c_uint16, [c_float]),
    ("ssf_f16_to_f32", c_float, [ctypes.c_uint16]),
]


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
        l = ctypes.CDLL(LIB_PATH)
        for name, res, args in _SIGS:
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _lib = l
    return _lib


class HipError(RuntimeError):
    pass


def _chk(rc, what="call"):
    if rc != 0:
        raise HipError(f"{what}: {lib().sml_hip_last_error().decode(errors='replace')}")


def init(device=0):
    why = ctypes.create_string_buffer(512)
    if not lib().sml_hip_init(device, why, 512):
        raise HipError(f"init: {lib().sml_hip_last_error().decode(errors='replace')}")


class DevBuf:
    """A device allocation owned by the library's HIP runtime."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = lib().sml_hip_malloc(max(1, self.nbytes))
        if not self.ptr:
            raise HipError(f"malloc: {lib().sml_hip_last_error().decode(errors='replace')}")

    @classmethod
    def of(cls, arr):
        a = np.ascontiguousarray(arr)
        b = cls(a.nbytes)
        b.write(a)
        return b

    def write(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _chk(lib().sml_hip_h2d(self.ptr, a.ctypes.data, a.nbytes), "h2d")

    def read(self, dtype, count=None):
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else int(count)
        out = np.empty(n, dtype=dtype)
        _chk(lib().sml_hip_d2h(out.ctypes.data, self.ptr, out.nbytes), "d2h")
        return out

    def zero(self):
        _chk(lib().sml_hip_memset(self.ptr, 0, self.nbytes), "memset")

    def free(self):
        if self.ptr:
            lib().sml_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Mat:
    """A quantized FLAT matrix resident in HBM."""

    def __init__(self, handle):
        if not handle:
            raise HipError(f"matrix upload: {lib().sml_hip_last_error().decode(errors='replace')}")
        self.h = handle
        r, c, b = c_int(), c_int(), c_int()
        lib().sml_hip_mat_info(handle, ctypes.byref(r), ctypes.byref(c), ctypes.byref(b))
        self.rows, self.cols, self.nbits = r.value, c.value, b.value
        self.bytes = lib().sml_hip_mat_bytes(handle)

    @classmethod
    def from_file(cls, path, name):
        return cls(lib().sml_hip_mat_from_file(str(path).encode(), name.encode()))

    @classmethod
    def from_q4k(cls, blocks, rows, cols):
        """GGUF Q4_K blocks (uint8, rows x cols/256 x 144 bytes) repacked into
        the FLAT Q4 layout and uploaded."""
        b = np.ascontiguousarray(blocks, np.uint8)
        if b.size != rows * (cols // 256) * 144:
            raise ValueError("Q4_K blocks do not match the shape")
        return cls(lib().sml_hip_mat_from_q4k(b.ctypes.data, rows, cols))

    @classmethod
    def from_q5k(cls, blocks, rows, cols):
        """GGUF Q5_K blocks (uint8, rows x cols/256 x 176 bytes) repacked into
        the FLAT Q5 layout and uploaded."""
        b = np.ascontiguousarray(blocks, np.uint8)
        if b.size != rows * (cols // 256) * 176:
            raise ValueError("Q5_K blocks do not match the shape")
        return cls(lib().sml_hip_mat_from_q5k(b.ctypes.data, rows, cols))

    def free(self):
        if self.h:
            lib().sml_hip_mat_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Act:
    """A quantized activation on the device: int8 codes, per-group scale and sum."""

    def __init__(self, n):
        self.n = n
        self.q = DevBuf(n)
        self.scale = DevBuf(n // 32 * 4)
        self.sums = DevBuf(n // 32 * 4)

    def read(self):
        return (self.q.read(np.int8), self.scale.read(np.float32), self.sums.read(np.int32))


def normq(x, act, perm=None, w=None, resid=None, eps=1e-6, per256=False):
    """Device RMSNorm (w given) + gather + int8 quantize of device vector x."""
    _chk(lib().sml_hip_normq(x.ptr, resid.ptr if resid else None, w.ptr if w else None, eps, act.n,
                             perm.ptr if perm else None, act.q.ptr, act.scale.ptr, act.sums.ptr,
                             1 if per256 else 0), "normq")


def matvec(m, act, y):
    _chk(lib().sml_hip_matvec(m.h, act.q.ptr, act.scale.ptr, act.sums.ptr, y.ptr), "matvec")


def matvec_swiglu(gate, up, act, h):
    _chk(lib().sml_hip_matvec_swiglu(gate.h, up.h, act.q.ptr, act.scale.ptr, act.sums.ptr, h.ptr), "swiglu")


def matvec_normq(m, x, y, w=None, perm=None, eps=1e-6):
    """y = W . quantize(gather(RMSNorm(x))), the activation computed in the GEMV's prologue."""
    _chk(lib().sml_hip_matvec_normq(m.h, x.ptr, w.ptr if w else None, eps, perm.ptr if perm else None, y.ptr),
         "matvec_normq")


def matvec_swiglu_fused(gate, up, h, x=None, w=None, perm=None, eps=1e-6, act=None, hact=None):
    """SwiGLU GEMV with the prologue fusion (x given) and/or h quantized into hact."""
    _chk(lib().sml_hip_matvec_swiglu_fused(
        gate.h, up.h, x.ptr if x else None, w.ptr if w else None, eps, perm.ptr if perm else None,
        act.q.ptr if act else None, act.scale.ptr if act else None, act.sums.ptr if act else None, h.ptr,
        hact.q.ptr if hact else None, hact.scale.ptr if hact else None, hact.sums.ptr if hact else None),
        "swiglu_fused")


def unpack(m, row0, nrows):
    out = DevBuf(max(1, nrows * m.cols))
    _chk(lib().sml_hip_unpack(m.h, row0, nrows, out.ptr), "unpack")
    return out.read(np.uint8, nrows * m.cols).reshape(nrows, m.cols)


def sync():
    _chk(lib().sml_hip_sync(), "sync")


def synth_model(path, n_layer, n_embd, n_head, n_head_kv, n_ff, n_vocab, n_ctx_train=4096,
                rope_theta=1e6, rms_eps=1e-6, nbits=4, tied=False, qkv_bias=False, random_perm=False,
                n_expert=0, n_expert_used=0, moe_flags=0, step_sigma=0.02, router_sigma=1.0 / 64, seed=1,
                zero_mean=True, moe_scale=0.0, moe_groups=0, moe_topk_group=0, exp_bias=False, n_ff_shexp=0,
                shexp_gate=False):
    """Write a seeded synthetic SSF decoder (sheep_amd/csrc/ssf.c). zero_mean
    puts every group's min at -(2^b - 1)/2 steps, so the uniform codes give
    weights of mean zero and the logits depend on the input; False keeps the
    single-GEMV recipe (min at -2^(b-1) steps). MoE files may carry the
    routing fields (moe_flags bits 0-3, moe_scale, moe_groups,
    moe_topk_group), a correction bias per layer (exp_bias) and a shared
    expert of width n_ff_shexp (with its sigmoid gate: shexp_gate)."""
    sp = SynthSpec(n_layer, n_embd, n_head, n_head_kv, n_ff, n_vocab, n_ctx_train, rope_theta, rms_eps,
                   nbits, int(tied), int(qkv_bias), int(random_perm), n_expert, n_expert_used, moe_flags,
                   step_sigma, router_sigma, seed, int(zero_mean), moe_scale, moe_groups, moe_topk_group,
                   int(exp_bias), n_ff_shexp, int(shexp_gate))
    why = ctypes.create_string_buffer(512)
    if not lib().ssf_synth_model(str(path).encode(), ctypes.byref(sp), why, 512):
        raise RuntimeError(why.value.decode())
    return path


def synth_matrix(path, rows, cols, nbits=4, random_perm=False, step_sigma=0.02, seed=1):
    """Write a seeded SSF file holding one quantized matrix named 'w'."""
    why = ctypes.create_string_buffer(512)
    if not lib().ssf_synth_matrix(str(path).encode(), rows, cols, nbits, int(random_perm), step_sigma, seed, why, 512):
        raise RuntimeError(why.value.decode())
    return path


class Decoder:
    """The sml-gpu.h forward pass: one model per process."""

    def __init__(self, path, n_ctx=4096, gpu_layers=0, exact=False):
        """exact: open in exact mode (SML_EXACT=1 for the open), where every
        kernel follows the reference CPU path's float order and the logits
        equal it bit for bit."""
        why = ctypes.create_string_buffer(1024)
        old = os.environ.get("SML_EXACT")
        os.environ["SML_EXACT"] = "1" if exact else "0"
        try:
            ok = lib().sml_gpu_open(str(path).encode(), n_ctx, 1, gpu_layers, why, 1024)
        finally:
            if old is None:
                del os.environ["SML_EXACT"]
            else:
                os.environ["SML_EXACT"] = old
        if not ok:
            raise HipError(f"sml_gpu_open: {why.value.decode(errors='replace')}")
        of = c_int()
        # layers whose matrices stay in HBM (a split streams the rest), of n_layer
        self.gpu_layers = lib().sml_gpu_layers(ctypes.byref(of))
        self.n_layer = of.value
        self.n_ctx = n_ctx
        self.exact = bool(lib().sml_gpu_exact())

    def prompt_mode(self, level):
        """How prefill reads a prompt: 0 a token at a time, 1 batched with
        every product the GEMV's arithmetic (the default), 2 batched with Q4
        products on MFMA."""
        lib().sml_gpu_prompt_mode(level)

    def step(self, tok, pos, n_vocab):
        p = lib().sml_gpu_step(tok, pos)
        if not p:
            raise HipError(f"sml_gpu_step: {lib().sml_gpu_last_error().decode(errors='replace')}")
        return np.ctypeslib.as_array(p, shape=(n_vocab,)).copy()

    def slots(self, ns):
        if lib().sml_gpu_slots(ns) != ns:
            raise HipError(f"sml_gpu_slots: {lib().sml_gpu_last_error().decode(errors='replace')}")

    def prefill_slot(self, slot, ids, pos0, n_vocab):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        p = lib().sml_gpu_prefill_slot(slot, a.ctypes.data_as(P(c_int)), pos0, len(a))
        if not p:
            raise HipError(f"sml_gpu_prefill_slot: {lib().sml_gpu_last_error().decode(errors='replace')}")
        return np.ctypeslib.as_array(p, shape=(n_vocab,)).copy()

    def step_multi(self, toks, poss, slots, n_vocab):
        t = np.ascontiguousarray(toks, np.int32)
        p = np.ascontiguousarray(poss, np.int32)
        s = np.ascontiguousarray(slots, np.int32)
        out = np.empty((len(t), n_vocab), np.float32)     # every entry is written
        if lib().sml_gpu_step_multi(t.ctypes.data_as(P(c_int)), p.ctypes.data_as(P(c_int)), s.ctypes.data_as(P(c_int)),
                                    len(t), out.ctypes.data) != len(t):
            raise HipError(f"sml_gpu_step_multi: {lib().sml_gpu_last_error().decode(errors='replace')}")
        return out

    def prefill(self, ids, pos0, n_vocab):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        p = lib().sml_gpu_prefill(a.ctypes.data_as(P(c_int)), pos0, len(a))
        if not p:
            raise HipError(f"sml_gpu_prefill: {lib().sml_gpu_last_error().decode(errors='replace')}")
        return np.ctypeslib.as_array(p, shape=(n_vocab,)).copy()

    def generate(self, tok, pos, n):
        out = np.zeros(n, dtype=np.int32)
        if lib().sml_gpu_generate(tok, pos, n, out.ctypes.data_as(P(c_int))) != n:
            raise HipError(f"sml_gpu_generate: {lib().sml_gpu_last_error().decode(errors='replace')}")
        return out

    def last_ms(self):
        return lib().sml_gpu_last_ms()

    def weight_bytes(self):
        return lib().sml_gpu_weight_bytes()

    def close(self):
        lib().sml_gpu_close()


class MoE:
    """One MoE FFN layer of an SSF file resident in HBM (sml_hip_moe_*)."""

    def __init__(self, path, layer=0, max_tokens=16):
        h = lib().sml_hip_moe_from_file(str(path).encode(), layer, max_tokens)
        if not h:
            raise HipError(f"moe: {lib().sml_hip_last_error().decode(errors='replace')}")
        self.h = h
        ne, k, nf, eb = c_int(), c_int(), c_int(), c_size_t()
        lib().sml_hip_moe_info(h, ctypes.byref(ne), ctypes.byref(k), ctypes.byref(nf), ctypes.byref(eb))
        self.nexp, self.k, self.n_ff, self.expert_bytes = ne.value, k.value, nf.value, eb.value

    def regime(self, per256):
        """Quantize the expert inputs per 256 values (True) or per 32 (False)."""
        _chk(lib().sml_hip_moe_regime(self.h, 1 if per256 else 0), "moe_regime")

    def ffn(self, x, T, out, sel=None, w=None, logits=None):
        _chk(lib().sml_hip_moe_ffn(self.h, x.ptr, T, out.ptr, sel.ptr if sel else None, w.ptr if w else None,
                                   logits.ptr if logits else None), "moe_ffn")

    def time(self, x, T, out, iters):
        ms = c_float()
        cnt = np.zeros(self.nexp, np.int32)
        _chk(lib().sml_hip_moe_time(self.h, x.ptr, T, out.ptr, iters, ctypes.byref(ms), cnt.ctypes.data), "moe_time")
        return ms.value, cnt

    def free(self):
        if self.h:
            lib().sml_hip_moe_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def gemm(m, act_q, act_s, act_u, nrow, y, per256=False):
    """y [nrow][rows] = W . a[r] for nrow activation rows (device buffers),
    quantized per 32 values (per256 False) or per 256 (True)."""
    f = lib().sml_hip_gemm_sb if per256 else lib().sml_hip_gemm
    _chk(f(m.h, act_q.ptr, act_s.ptr, act_u.ptr, nrow, y.ptr), "gemm")


def gemm_swiglu(gate, up, act_q, act_s, act_u, nrow, h, per256=False):
    f = lib().sml_hip_gemm_swiglu_sb if per256 else lib().sml_hip_gemm_swiglu
    _chk(f(gate.h, up.h, act_q.ptr, act_s.ptr, act_u.ptr, nrow, h.ptr), "gemm_swiglu")


def q4k_repack(blocks, rows, cols):
    """The host repack of GGUF Q4_K blocks into FLAT Q4 arrays (no GPU):
    (plane [rows][cols/2], sd, md [rows][cols/256] fp16 bits, sq, mq [rows][cols/32])."""
    b = np.ascontiguousarray(blocks, np.uint8)
    nb = cols // 256
    plane = np.zeros((rows, cols // 2), np.uint8)
    sd = np.zeros((rows, nb), np.uint16)
    md = np.zeros((rows, nb), np.uint16)
    sq = np.zeros((rows, cols // 32), np.uint8)
    mq = np.zeros((rows, cols // 32), np.uint8)
    if lib().sml_hip_q4k_repack(b.ctypes.data, rows, cols, plane.ctypes.data, sd.ctypes.data, sq.ctypes.data,
                                md.ctypes.data, mq.ctypes.data) != 0:
        raise ValueError("Q4_K blocks do not match the shape")
    return plane, sd, md, sq, mq


def q5k_repack(blocks, rows, cols):
    """The host repack of GGUF Q5_K blocks into FLAT Q5 arrays (no GPU):
    ([4-bit plane [rows][cols/2], 1-bit plane [rows][cols/8]], sd, md
    [rows][cols/256] fp16 bits, sq, mq [rows][cols/32])."""
    b = np.ascontiguousarray(blocks, np.uint8)
    nb = cols // 256
    p4 = np.zeros((rows, cols // 2), np.uint8)
    p1 = np.zeros((rows, cols // 8), np.uint8)
    sd = np.zeros((rows, nb), np.uint16)
    md = np.zeros((rows, nb), np.uint16)
    sq = np.zeros((rows, cols // 32), np.uint8)
    mq = np.zeros((rows, cols // 32), np.uint8)
    if b.size != rows * nb * 176 or lib().sml_hip_q5k_repack(b.ctypes.data, rows, cols, p4.ctypes.data,
                                                              p1.ctypes.data, sd.ctypes.data, sq.ctypes.data,
                                                              md.ctypes.data, mq.ctypes.data) != 0:
        raise ValueError("Q5_K blocks do not match the shape")
    return [p4, p1], sd, md, sq, mq
