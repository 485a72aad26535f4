"""CPU ORACLE -- test infrastructure only.

ctypes bindings for the plain-C restatement (liboracle.so) and, where it was
built, the reference engine's own CPU path (_ref/libsmlref.so). Only tests/,
__graft_entry__.smoke() and bench.py's CPU-baseline leg load this module, as
the checker or the reported CPU baseline.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libsmlref.so")

c_int, c_float, c_void_p, c_char_p, c_uint = ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_char_p, ctypes.c_uint
P = ctypes.POINTER


class OrcTensor(ctypes.Structure):
    _fields_ = [("plane", c_void_p * 4), ("sd", c_void_p), ("sq", c_void_p), ("md", c_void_p), ("mq", c_void_p),
                ("rows", c_int), ("cols", c_int), ("nbits", c_int), ("scale6", c_int), ("minneg", c_int)]


class SmlAct(ctypes.Structure):
    """The reference's sml_act (sml/sml-kernel.h:128-134)."""
    _fields_ = [("q", c_void_p), ("scale", c_void_p), ("sums", c_void_p), ("n", c_int)]


_orc = None
_ref = None


def oracle():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_PATH):
            raise RuntimeError(f"{ORACLE_PATH} is not built (make -C oracle)")
        l = ctypes.CDLL(ORACLE_PATH)
        sig = {
            "orc_quantize_act": (None, [c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
            "orc_quantize_act_sb": (None, [c_void_p, c_int, c_void_p, c_void_p, c_void_p]),
            "orc_unpack_row": (None, [P(OrcTensor), c_int, c_void_p]),
            "orc_dequant_row": (None, [P(OrcTensor), c_int, c_void_p]),
            "orc_step": (c_float, [P(OrcTensor), c_int, c_int]),
            "orc_min": (c_float, [P(OrcTensor), c_int, c_int]),
            "orc_matvec": (None, [P(OrcTensor), c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int]),
            "orc_rms_norm": (None, [c_void_p, c_void_p, c_void_p, c_int, c_float]),
            "orc_rope_table": (None, [c_float, c_int, c_int, c_void_p, c_void_p]),
            "orc_rope": (None, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p]),
            "orc_f32_to_f16": (ctypes.c_uint16, [c_float]),
            "orc_f16_to_f32": (c_float, [ctypes.c_uint16]),
            "orc_attn_head": (None, [c_void_p, c_void_p, c_void_p, ctypes.c_size_t, c_int, c_int, c_float, c_void_p, c_void_p]),
            "orc_silu_mul": (None, [c_void_p, c_void_p, c_int]),
            "orc_moe_route": (c_int, [c_void_p, c_int, c_int, c_uint, c_void_p, c_void_p]),
            "orc_moe_route2": (c_int, [c_void_p, c_int, c_int, c_uint, c_float, c_int, c_int, c_void_p, c_void_p,
                                       c_void_p]),
            "orc_router": (None, [c_void_p, c_void_p, c_int, c_int, c_void_p]),
            "orc_argmax": (c_int, [c_void_p, c_int]),
            "orc_expf_published": (c_float, [c_float]),
            "orc_q4k_dequant_row": (None, [c_void_p, c_int, c_void_p]),
            "orc_q5k_dequant_row": (None, [c_void_p, c_int, c_void_p]),
            "orc_gguf_dequant_f16_row": (c_int, [c_int, c_void_p, c_int, c_void_p]),
            "orc_gptq_dequant_row_gidx": (None, [c_void_p] * 4 + [c_int] * 5 + [c_void_p]),
            "orc_gptq_matvec_gidx": (None, [c_void_p] * 4 + [c_int] * 4 + [c_void_p, c_void_p]),
            "orc_expf_mismatches": (ctypes.c_long, [ctypes.c_uint]),
            "orc_gptq_unpack_row": (None, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
            "orc_gptq_dequant_row": (None, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p]),
            "orc_gptq_matvec": (None, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
            "orc_awq_unpack_row": (None, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
            "orc_awq_dequant_row": (None, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]),
            "orc_model_open": (c_void_p, [c_char_p, c_int]),
            "orc_model_close": (None, [c_void_p]),
            "orc_forward": (P(c_float), [c_void_p, c_int, c_int]),
            "orc_n_vocab": (c_int, [c_void_p]),
            "orc_model_per256": (None, [c_void_p, c_int]),
            "orc_asym_grid": (None, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int, c_int,
                                     c_int, c_void_p, c_void_p]),
            "orc_field_search": (None, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                        c_int, c_int, c_int, c_void_p, c_int]),
            "orc_grid_facs": (c_int, [c_int, c_void_p]),
            "orc_two_level": (None, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p]),
            "orc_requant_codes": (None, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p]),
            "orc_perm_maxabs": (None, [c_void_p, c_int, c_int, c_void_p]),
            "orc_unpack_dequant_f16": (None, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                              c_int, c_int, c_void_p]),
            "orc_requant": (None, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                                   c_void_p, c_void_p, c_void_p, c_void_p]),
        }
        for k, (r, a) in sig.items():
            f = getattr(l, k)
            f.restype, f.argtypes = r, a
        _orc = l
    return _orc


REFQ_PATH = os.path.join(HERE, "_ref", "libsmlquant.so")
_refq = None


def have_refq():
    return os.path.exists(REFQ_PATH)


def refq():
    """The reference quantizer's fused C searches (sml/sml-quant.c), compiled from its source."""
    global _refq
    if _refq is None:
        if not have_refq():
            raise RuntimeError(f"{REFQ_PATH} is not built (its sources are only present where the reference is)")
        l = ctypes.CDLL(REFQ_PATH)
        l.sml_asym_grid.restype = None
        l.sml_asym_grid.argtypes = [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int, c_int,
                                    c_int, c_void_p, c_void_p]
        l.sml_field_search.restype = None
        l.sml_field_search.argtypes = [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                       c_int, c_int, c_int, c_void_p, c_int]
        _refq = l
    return _refq


def _pp(a):
    return None if a is None else a.ctypes.data


def grid_facs(ncand=20):
    f = np.zeros(max(64, ncand + 4), np.float32)
    n = oracle().orc_grid_facs(ncand, f.ctypes.data)
    return f[:n].copy()


def asym_grid(wp, group, nbits, wt=None, rem=0, ncand=20, iters=3, refit=1, lib=None):
    """(mins, steps) [rows][cols/group] from the oracle, or from the
    reference's own library when lib is refq()."""
    wp = np.ascontiguousarray(wp, np.float32)
    rows, cols = wp.shape
    facs = grid_facs(ncand)
    ol = np.zeros((rows, cols // group), np.float32)
    os_ = np.zeros_like(ol)
    wt = None if wt is None else np.ascontiguousarray(wt, np.float32)
    if lib is None:
        oracle().orc_asym_grid(wp.ctypes.data, rows, cols, group, nbits, rem, _pp(wt), facs.ctypes.data, len(facs),
                               iters, refit, ol.ctypes.data, os_.ctypes.data)
    else:
        lib.sml_asym_grid(wp.ctypes.data, rows, cols, group, nbits, rem, _pp(wt), facs.ctypes.data, len(facs),
                          iters, refit, ol.ctypes.data, os_.ctypes.data)
    return ol, os_


def field_search(w, dv, dm, q8, mq8, group, nmax, hi=255, moff=127, mmax=254, wt=None, radius=2, lib=None):
    """(q8, mq8) int32 after the field search, from the oracle or the reference's library."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    a = np.ascontiguousarray(q8, np.int32).copy()
    b = np.ascontiguousarray(mq8, np.int32).copy()
    dv = np.ascontiguousarray(dv, np.float32)
    dm = np.ascontiguousarray(dm, np.float32)
    wt = None if wt is None else np.ascontiguousarray(wt, np.float32)
    f = oracle().orc_field_search if lib is None else lib.sml_field_search
    f(w.ctypes.data, rows, cols, group, dv.ctypes.data, dm.ctypes.data, a.ctypes.data, b.ctypes.data, nmax, hi,
      moff, mmax, _pp(wt), radius)
    return a, b


def two_level(v, gps=8, signed=False):
    """(d16 uint16 [rows][nsb], q8 uint8 [rows][ng], eff float32 [rows][ng])."""
    v = np.ascontiguousarray(v, np.float32)
    rows, ng = v.shape
    nsb = (ng + gps - 1) // gps
    d16 = np.zeros((rows, nsb), np.uint16)
    q8 = np.zeros((rows, ng), np.uint8)
    eff = np.zeros((rows, ng), np.float32)
    oracle().orc_two_level(v.ctypes.data, rows, ng, gps, int(signed), d16.ctypes.data, q8.ctypes.data, eff.ctypes.data)
    return d16, q8, eff


def perm_maxabs(w):
    w = np.ascontiguousarray(w, np.float32)
    p = np.zeros(w.shape[1], np.int32)
    oracle().orc_perm_maxabs(w.ctypes.data, w.shape[0], w.shape[1], p.ctypes.data)
    return p


def unpack_dequant_f16(qweight, qzeros, scales, g_idx, rows, cols, bits, group, zero_add=1, awq=False):
    """[rows][cols] float32 holding the fp16 values of the unpacked copy."""
    out = np.zeros((rows, cols), np.float32)
    qw = np.ascontiguousarray(qweight, np.int32)
    qz = None if qzeros is None else np.ascontiguousarray(qzeros, np.int32)
    sc = np.ascontiguousarray(scales, np.float16).view(np.uint16)
    gi = None if g_idx is None else np.ascontiguousarray(g_idx, np.int32)
    oracle().orc_unpack_dequant_f16(qw.ctypes.data, _pp(qz), sc.ctypes.data, _pp(gi), rows, cols, bits, group,
                                    zero_add, int(awq), out.ctypes.data)
    return out


def requant(w, nbits=4, perm=None, wt=None, radius=2):
    """The oracle's whole re-quantization: dict of codes [rows][cols] (permuted
    order), sd, sq, md, mq, perm."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    ng, ns = cols // 32, cols // 256
    out = {"codes": np.zeros((rows, cols), np.uint8), "sd": np.zeros((rows, ns), np.uint16),
           "sq": np.zeros((rows, ng), np.uint8), "md": np.zeros((rows, ns), np.uint16),
           "mq": np.zeros((rows, ng), np.uint8), "perm": np.zeros(cols, np.int32)}
    pin = None if perm is None else np.ascontiguousarray(perm, np.int32)
    wt = None if wt is None else np.ascontiguousarray(wt, np.float32)
    oracle().orc_requant(w.ctypes.data, rows, cols, nbits, _pp(pin), _pp(wt), radius, out["codes"].ctypes.data,
                         out["sd"].ctypes.data, out["sq"].ctypes.data, out["md"].ctypes.data, out["mq"].ctypes.data,
                         out["perm"].ctypes.data)
    return out


def have_ref():
    return os.path.exists(REF_PATH)


def ref():
    """The reference's own CPU path, compiled from its sources (oracle/Makefile)."""
    global _ref
    if _ref is None:
        if not have_ref():
            raise RuntimeError(f"{REF_PATH} is not built (its sources are only present where the reference is)")
        l = ctypes.CDLL(REF_PATH)
        sig = {
            "ref_layout": (None, [P(ctypes.c_long)]),
            "ref_open": (c_void_p, [c_char_p, c_int, c_int, c_int]),
            "ref_close": (None, [c_void_p]),
            "ref_forward": (P(c_float), [c_void_p, c_int, c_int]),
            "ref_prefill": (P(c_float), [c_void_p, c_void_p, c_int, c_int]),
            "ref_n_vocab": (c_int, [c_void_p]),
            "ref_moe_route": (c_int, [c_void_p, c_int, c_int, c_uint, c_void_p, c_void_p]),
            "ref_moe_route2": (c_int, [c_void_p, c_int, c_int, c_uint, c_float, c_int, c_int, c_void_p, c_void_p,
                                       c_void_p]),
            "sml_quantize_act": (None, [P(SmlAct), c_void_p, c_int]),
            "sml_quantize_act_sb": (None, [P(SmlAct), c_void_p, c_int]),
            "sml_matvec_rows_flat4": (None, [c_void_p] * 6 + [P(SmlAct), c_int, c_int, c_int]),
            "sml_matvec_rows_flat6": (None, [c_void_p] * 7 + [P(SmlAct), c_int, c_int, c_int]),
            "sml_matvec_rows_flat8": (None, [c_void_p] * 7 + [P(SmlAct), c_int, c_int, c_int]),
            "sml_matvec_rows": (None, [c_void_p] * 6 + [P(SmlAct), c_int, c_int, c_int, c_int, c_float]),
            "sml_matvec_bits1": (None, [c_void_p] * 4 + [P(SmlAct), c_int, c_int, c_int, c_int, c_int, c_int]),
            "sml_dequant_row": (None, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int]),
            "sml_dequant_row_flat4": (None, [c_void_p] * 6 + [c_int, c_int]),
            "sml_dequant_row_flat6": (None, [c_void_p] * 7 + [c_int, c_int]),
            "sml_dequant_row_flat8": (None, [c_void_p] * 7 + [c_int, c_int]),
            "sml_dequant_bits1_add": (None, [c_void_p] * 4 + [c_int, c_int, c_int]),
            "sml_matvec_batch_flat4": (None, [c_void_p] * 6 + [c_void_p, c_int, c_int, c_int, c_int, c_int]),
            "sml_matvec_batch_flat4_sb": (None, [c_void_p] * 6 + [c_void_p, c_int, c_int, c_int, c_int, c_int]),
            "sml_matvec_batch_flat6_sb": (None, [c_void_p] * 7 + [c_void_p, c_int, c_int, c_int, c_int, c_int]),
            "sml_rlp_ok": (c_int, [c_int, c_int, c_int, c_int]),
            "sml_rlp_bytes": (ctypes.c_size_t, [c_int, c_int, c_int]),
            "sml_rlp_pack": (None, [c_void_p] * 7 + [c_int, c_int, c_int, c_int]),
            "sml_rlp_matvec": (None, [c_void_p, c_int, c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int]),
            "ref_multi_open": (c_void_p, [c_char_p, c_int, c_int, c_int]),
            "ref_multi_forward": (P(c_float), [c_void_p, c_int, c_int, c_int]),
            "ref_multi_step": (None, [c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
            "ref_multi_close": (None, [c_void_p]),
            "sml_kernel_init": (None, []),
            "sml_kernel_scale6": (None, [c_int]),
            "sml_kernel_minneg": (None, [c_int]),
        }
        for k, (r, a) in sig.items():
            f = getattr(l, k)
            f.restype, f.argtypes = r, a
        l.sml_kernel_init()
        _ref = l
    return _ref


def ptr(a):
    return None if a is None else a.ctypes.data


def tensor_view(t):
    """OrcTensor over an sheep_amd.ssf.Tensor's arrays (kept alive by the caller)."""
    ot = OrcTensor()
    pl = t.planes()
    for i, p in enumerate(pl):
        ot.plane[i] = p.ctypes.data
    ot.sd, ot.sq = t.sd.ctypes.data, t.sq.ctypes.data
    ot.md = t.md.ctypes.data if t.md is not None else None
    ot.mq = t.mq.ctypes.data if t.mq is not None else None
    ot.rows, ot.cols, ot.nbits = t.rows, t.cols, t.nbits
    six = (t.f.hdr["flags"] & 2) != 0
    ot.scale6, ot.minneg = int(six), int(six and (t.f.hdr["flags"] & 4) != 0)
    return ot


def quantize_act(x, per256=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = len(x)
    q = np.zeros(n, np.int8)
    s = np.zeros(n // 32, np.float32)
    u = np.zeros(n // 32, np.int32)
    f = oracle().orc_quantize_act_sb if per256 else oracle().orc_quantize_act
    f(x.ctypes.data, n, q.ctypes.data, s.ctypes.data, u.ctypes.data)
    return q, s, u


def ref_quantize_act(x, per256=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = len(x)
    q = np.zeros(n, np.int8)
    s = np.zeros(n // 32, np.float32)
    u = np.zeros(n // 32, np.int32)
    a = SmlAct(q.ctypes.data, s.ctypes.data, u.ctypes.data, n)
    (ref().sml_quantize_act_sb if per256 else ref().sml_quantize_act)(ctypes.byref(a), x.ctypes.data, n)
    return q, s, u


def unpack(t, row):
    ot = tensor_view(t)
    out = np.zeros(t.cols, np.uint8)
    oracle().orc_unpack_row(ctypes.byref(ot), row, out.ctypes.data)
    return out


def dequant_row(t, row):
    ot = tensor_view(t)
    out = np.zeros(t.cols, np.float32)
    oracle().orc_dequant_row(ctypes.byref(ot), row, out.ctypes.data)
    return out


def matvec(t, q, s, u, row0=0, row1=None):
    row1 = t.rows if row1 is None else row1
    ot = tensor_view(t)
    y = np.zeros(t.rows, np.float32)
    oracle().orc_matvec(ctypes.byref(ot), q.ctypes.data, s.ctypes.data, u.ctypes.data, y.ctypes.data, row0, row1)
    return y


def ref_matvec(t, q, s, u):
    """y = W.x through the reference's own kernels, dispatched as issue_rows_act
    does (sml/sml-run.c:612-680)."""
    r = ref()
    a = SmlAct(q.ctypes.data, s.ctypes.data, u.ctypes.data, len(q))
    y = np.zeros(t.rows, np.float32)
    pl = t.planes()
    md = t.md.ctypes.data if t.md is not None else None
    mq = t.mq.ctypes.data if t.mq is not None else None
    sd, sq = t.sd.ctypes.data, t.sq.ctypes.data
    R, n, nb = t.rows, t.cols, t.nbits
    yp = y.ctypes.data
    ab = ctypes.byref(a)
    if nb == 4:
        r.sml_matvec_rows_flat4(yp, pl[0].ctypes.data, sd, sq, md, mq, ab, 0, R, n)
    elif nb == 2:
        r.sml_matvec_rows(yp, pl[0].ctypes.data, sd, sq, md, mq, ab, 0, R, n, 0, 0.0)
    elif nb == 3:
        r.sml_matvec_rows(yp, pl[0].ctypes.data, sd, sq, md, mq, ab, 0, R, n, 0, 0.0)
        r.sml_matvec_bits1(yp, pl[1].ctypes.data, sd, sq, ab, 1, 0, 0, R, n, 2)
    elif nb == 5:
        r.sml_matvec_rows_flat4(yp, pl[0].ctypes.data, sd, sq, md, mq, ab, 0, R, n)
        r.sml_matvec_bits1(yp, pl[1].ctypes.data, sd, sq, ab, 1, 0, 0, R, n, 4)
    elif nb == 6:
        r.sml_matvec_rows_flat6(yp, pl[1].ctypes.data, pl[0].ctypes.data, sd, sq, md, mq, ab, 0, R, n)
    elif nb == 7:
        r.sml_matvec_rows_flat6(yp, pl[0].ctypes.data, pl[1].ctypes.data, sd, sq, md, mq, ab, 0, R, n)
        r.sml_matvec_bits1(yp, pl[2].ctypes.data, sd, sq, ab, 1, 0, 0, R, n, 6)
    elif nb == 8:
        r.sml_matvec_rows_flat8(yp, pl[0].ctypes.data, pl[1].ctypes.data, sd, sq, md, mq, ab, 0, R, n)
    return y


def _acts(q, s, u):
    """An array of the reference's sml_act over rows of q [nb][n], s/u [nb][n/32]."""
    nb, n = q.shape
    arr = (SmlAct * nb)()
    for i in range(nb):
        arr[i] = SmlAct(q[i].ctypes.data, s[i].ctypes.data, u[i].ctypes.data, n)
    return arr


def ref_matvec_batch(t, q, s, u, sb=True):
    """y [nb][rows] through the reference's batched flat 4-bit kernel:
    sml_matvec_batch_flat4_sb on per-256 activations (sb) or
    sml_matvec_batch_flat4 on per-32 ones (sml/sml-kernel.c:1008-1021,1414-1435);
    a 6-bit tensor through sml_matvec_batch_flat6_sb (per-256 only,
    sml/sml-kernel.c:1604-1619: the 4-bit plane's and the 2-bit plane's parts)."""
    q, s, u = (np.ascontiguousarray(v) for v in (q, s, u))
    nb = q.shape[0]
    y = np.zeros((nb, t.rows), np.float32)
    pl = t.planes()
    md = t.md.ctypes.data if t.md is not None else None
    mq = t.mq.ctypes.data if t.mq is not None else None
    arr = _acts(q, s, u)
    if t.nbits == 6:
        if not sb:
            raise ValueError("the reference's 6-bit batch kernel takes per-256 activations")
        # the file's planes: [0] the 2-bit plane (code bits 4-5), [1] the 4-bit plane
        ref().sml_matvec_batch_flat6_sb(y.ctypes.data, pl[1].ctypes.data, pl[0].ctypes.data, t.sd.ctypes.data,
                                        t.sq.ctypes.data, md, mq, ctypes.addressof(arr), nb, t.rows, 0, t.rows, t.cols)
        return y
    f = ref().sml_matvec_batch_flat4_sb if sb else ref().sml_matvec_batch_flat4
    f(y.ctypes.data, pl[0].ctypes.data, t.sd.ctypes.data, t.sq.ctypes.data, md, mq, ctypes.addressof(arr), nb,
      t.rows, 0, t.rows, t.cols)
    return y


def ref_rlp_matvec(t, q, s, u):
    """y [nb][rows] through the reference's once-packed rows-in-lanes kernel
    (sml_rlp_pack + sml_rlp_matvec, sml/sml-kernel.c:1646-1840), the default
    multi-sequence path; per-256 activations. None when the tensor does not
    qualify (sml_rlp_ok)."""
    r = ref()
    if not r.sml_rlp_ok(t.rows, t.cols, t.nbits, int(t.mq is not None)):
        return None
    q, s, u = (np.ascontiguousarray(v) for v in (q, s, u))
    nb = q.shape[0]
    pk = np.zeros(r.sml_rlp_bytes(t.rows, t.cols, t.nbits), np.uint8)
    pl = t.planes()
    r.sml_rlp_pack(pk.ctypes.data, pl[0].ctypes.data, None, t.sd.ctypes.data, t.sq.ctypes.data, t.md.ctypes.data,
                   t.mq.ctypes.data, t.nbits, 0, t.rows // 8, t.cols)
    y = np.zeros((nb, t.rows), np.float32)
    arr = _acts(q, s, u)
    r.sml_rlp_matvec(y.ctypes.data, t.rows, pk.ctypes.data, t.nbits, ctypes.addressof(arr), nb, 0, t.rows, t.cols)
    return y


def ref_dequant_row(t, row):
    """One row through the reference's own dequantizers (sml/sml-run.c:586-603,3300-3335)."""
    r = ref()
    out = np.zeros(t.cols, np.float32)
    pl = t.planes()
    md = t.md.ctypes.data if t.md is not None else None
    mq = t.mq.ctypes.data if t.mq is not None else None
    sd, sq, n, nb, o = t.sd.ctypes.data, t.sq.ctypes.data, t.cols, t.nbits, out.ctypes.data
    if nb in (2, 3):
        arr = (c_void_p * 1)(pl[0].ctypes.data)
        r.sml_dequant_row(o, arr, 1, 1, sd, sq, md, mq, row, n)
        if nb == 3:
            r.sml_dequant_bits1_add(o, pl[1].ctypes.data, sd, sq, row, n, 2)
    elif nb in (4, 5):
        r.sml_dequant_row_flat4(o, pl[0].ctypes.data, sd, sq, md, mq, row, n)
        if nb == 5:
            r.sml_dequant_bits1_add(o, pl[1].ctypes.data, sd, sq, row, n, 4)
    elif nb == 6:
        r.sml_dequant_row_flat6(o, pl[1].ctypes.data, pl[0].ctypes.data, sd, sq, md, mq, row, n)
    elif nb == 7:
        r.sml_dequant_row_flat6(o, pl[0].ctypes.data, pl[1].ctypes.data, sd, sq, md, mq, row, n)
        r.sml_dequant_bits1_add(o, pl[2].ctypes.data, sd, sq, row, n, 6)
    elif nb == 8:
        r.sml_dequant_row_flat8(o, pl[0].ctypes.data, pl[1].ctypes.data, sd, sq, md, mq, row, n)
    return out


class OracleModel:
    """orc_forward over an SSF file."""

    def __init__(self, path, n_ctx, per256=False):
        self.h = oracle().orc_model_open(str(path).encode(), n_ctx)
        if not self.h:
            raise RuntimeError(f"oracle cannot open {path}")
        self.n_vocab = oracle().orc_n_vocab(self.h)
        self.per256(per256)

    def per256(self, on):
        """Quantize every product's input per 256 values (True) or per 32."""
        oracle().orc_model_per256(self.h, 1 if on else 0)

    def forward(self, tok, pos):
        p = oracle().orc_forward(self.h, tok, pos)
        return np.ctypeslib.as_array(p, shape=(self.n_vocab,)).copy()

    def close(self):
        if self.h:
            oracle().orc_model_close(self.h)
            self.h = None


class RefModel:
    """The reference's sml_forward / sml_prefill over an SSF file."""

    def __init__(self, path, n_ctx, threads=8):
        self.h = ref().ref_open(str(path).encode(), n_ctx, threads, 1)
        if not self.h:
            raise RuntimeError(f"the reference cannot open {path}")
        self.n_vocab = ref().ref_n_vocab(self.h)

    def forward(self, tok, pos):
        p = ref().ref_forward(self.h, tok, pos)
        return np.ctypeslib.as_array(p, shape=(self.n_vocab,)).copy()

    def prefill(self, ids, pos0):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        p = ref().ref_prefill(self.h, a.ctypes.data, pos0, len(a))
        return np.ctypeslib.as_array(p, shape=(self.n_vocab,)).copy()

    def close(self):
        if self.h:
            ref().ref_close(self.h)
            self.h = None


class RefMulti:
    """ns contexts of the reference engine over one SSF file: slots stepped
    one at a time (sml_forward) and together (sml_forward_multi)."""

    def __init__(self, path, n_ctx, ns, threads=8):
        self.h = ref().ref_multi_open(str(path).encode(), n_ctx, threads, ns)
        if not self.h:
            raise RuntimeError(f"the reference cannot open {path}")
        self.ns = ns
        hh = ref().ref_open(str(path).encode(), 0, 1, 0)
        self.n_vocab = ref().ref_n_vocab(hh)
        ref().ref_close(hh)

    def forward(self, slot, tok, pos):
        p = ref().ref_multi_forward(self.h, slot, tok, pos)
        return np.ctypeslib.as_array(p, shape=(self.n_vocab,)).copy()

    def step(self, toks, pos):
        ns = len(toks)
        t = np.ascontiguousarray(toks, dtype=np.int32)
        p = np.ascontiguousarray(pos, dtype=np.int32)
        out = np.zeros((ns, self.n_vocab), np.float32)
        ref().ref_multi_step(self.h, t.ctypes.data, p.ctypes.data, ns, out.ctypes.data)
        return out

    def close(self):
        if self.h:
            ref().ref_multi_close(self.h)
            self.h = None


# ------------------------------------------------------------ GPTQ-style 4-bit

def gptq_unpack_row(qweight, qzeros, rows, cols, row, group=128, zero_add=1):
    c = np.zeros(cols, np.uint8)
    z = np.zeros(cols // group, np.uint8)
    oracle().orc_gptq_unpack_row(ptr(qweight), ptr(qzeros), rows, cols, group, zero_add, row, ptr(c), ptr(z))
    return c, z


def gptq_dequant_row(qweight, qzeros, scales, rows, cols, row, group=128, zero_add=1):
    out = np.zeros(cols, np.float32)
    oracle().orc_gptq_dequant_row(ptr(qweight), ptr(qzeros), ptr(scales), rows, cols, group, zero_add, row, ptr(out))
    return out


def gptq_matvec(qweight, qzeros, scales, rows, cols, x, group=128, zero_add=1):
    y = np.zeros(rows, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    oracle().orc_gptq_matvec(ptr(qweight), ptr(qzeros), ptr(scales), rows, cols, group, zero_add, ptr(x), ptr(y))
    return y


def gptq_dequant_row_gidx(qweight, qzeros, scales, g_idx, rows, cols, row, group=128, zero_add=1):
    out = np.zeros(cols, np.float32)
    oracle().orc_gptq_dequant_row_gidx(ptr(qweight), ptr(qzeros), ptr(scales), ptr(g_idx), rows, cols, group,
                                       zero_add, row, ptr(out))
    return out


def gptq_matvec_gidx(qweight, qzeros, scales, g_idx, rows, cols, x, group=128, zero_add=1):
    y = np.zeros(rows, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    oracle().orc_gptq_matvec_gidx(ptr(qweight), ptr(qzeros), ptr(scales), ptr(g_idx), rows, cols, group, zero_add,
                                  ptr(x), ptr(y))
    return y


# ------------------------------------------------------------ AWQ 4-bit

def awq_unpack_row(qweight, qzeros, rows, cols, row, group=128):
    c = np.zeros(cols, np.uint8)
    z = np.zeros(cols // group, np.uint8)
    oracle().orc_awq_unpack_row(ptr(qweight), ptr(qzeros), rows, cols, group, row, ptr(c), ptr(z))
    return c, z


def awq_dequant_row(qweight, qzeros, scales, rows, cols, row, group=128):
    out = np.zeros(cols, np.float32)
    oracle().orc_awq_dequant_row(ptr(qweight), ptr(qzeros), ptr(scales), rows, cols, group, row, ptr(out))
    return out


def q4k_dequant(blocks, rows, cols):
    """GGUF Q4_K blocks [rows][cols/256][144] to float32 weights [rows][cols]
    by the published formula (orc_q4k_dequant_row)."""
    bl = np.ascontiguousarray(blocks, np.uint8).reshape(rows, -1)
    out = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        oracle().orc_q4k_dequant_row(bl[r].ctypes.data, cols, out[r].ctypes.data)
    return out


def q4k_pack_scales(sc, m):
    """The 12 scale bytes of a Q4_K block from eight 6-bit scales and mins, as
    ggml's quantizer packs them: sub-blocks 0-3 in the low six bits of bytes
    j (scale) and j+4 (min); 4-7 in the nibbles of byte j+4, their high two
    bits in the top bits of bytes j-4 (scale) and j (min)."""
    out = [0] * 12
    for j in range(8):
        s, n = int(sc[j]), int(m[j])
        if j < 4:
            out[j] |= s
            out[j + 4] |= n
        else:
            out[j + 4] = (s & 15) | ((n & 15) << 4)
            out[j - 4] |= (s >> 4) << 6
            out[j] |= (n >> 4) << 6
    return np.array(out, np.uint8)


def q4k_random_blocks(rows, cols, seed):
    """Random Q4_K blocks: d, dmin small positive fp16, 6-bit scales and mins,
    uniform codes."""
    rng = np.random.default_rng(seed)
    nb = rows * (cols // 256)
    blk = np.zeros((nb, 144), np.uint8)
    d = (np.abs(rng.standard_normal(nb)) * 0.002 + 1e-4).astype(np.float16)
    dm = (np.abs(rng.standard_normal(nb)) * 0.002 + 1e-4).astype(np.float16)
    blk[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = dm.view(np.uint8).reshape(nb, 2)
    for i in range(nb):
        blk[i, 4:16] = q4k_pack_scales(rng.integers(0, 64, 8), rng.integers(0, 64, 8))
    blk[:, 16:] = rng.integers(0, 256, (nb, 128), dtype=np.uint8)
    return blk.reshape(rows, cols // 256, 144)


GGUF_BLOCK = {8: (32, 34), 2: (32, 18), 14: (256, 210)}   # ggml type: (weights, bytes) per block


def gguf_dequant_f16(gtype, blocks, rows, cols):
    """GGUF Q8_0 (8), Q4_0 (2) or Q6_K (14) blocks [rows][cols/qk][bytes] to
    float32 [rows][cols] holding the fp16 copy (orc_gguf_dequant_f16_row)."""
    bl = np.ascontiguousarray(blocks, np.uint8).reshape(rows, -1)
    out = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        if oracle().orc_gguf_dequant_f16_row(gtype, bl[r].ctypes.data, cols, out[r].ctypes.data) != 0:
            raise ValueError(f"ggml type {gtype} at {cols} columns")
    return out


def q5k_dequant(blocks, rows, cols):
    """GGUF Q5_K blocks [rows][cols/256][176] to float32 weights [rows][cols]
    by the published formula (orc_q5k_dequant_row)."""
    bl = np.ascontiguousarray(blocks, np.uint8).reshape(rows, -1)
    out = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        oracle().orc_q5k_dequant_row(bl[r].ctypes.data, cols, out[r].ctypes.data)
    return out


def q5k_random_blocks(rows, cols, seed):
    """Random Q5_K blocks: Q4_K's fields drawn as in q4k_random_blocks, then
    random fifth bits (qh) and low nibbles."""
    rng = np.random.default_rng(seed)
    k4 = q4k_random_blocks(rows, cols, seed).reshape(-1, 144)
    nb = k4.shape[0]
    blk = np.zeros((nb, 176), np.uint8)
    blk[:, 0:16] = k4[:, 0:16]
    blk[:, 16:48] = rng.integers(0, 256, (nb, 32), dtype=np.uint8)
    blk[:, 48:] = rng.integers(0, 256, (nb, 128), dtype=np.uint8)
    return blk.reshape(rows, cols // 256, 176)


class FlatView:
    """An OrcTensor over raw FLAT arrays (the plane, or the list of planes of
    width nbits, sd, md, sq, mq as numpy arrays, kept alive here), e.g. a
    repacked Q4_K matrix or a re-quantized tensor."""

    def __init__(self, plane, sd, md, sq, mq, rows, cols, nbits=4):
        planes = list(plane) if isinstance(plane, (list, tuple)) else [plane]
        self.arrays = [np.ascontiguousarray(a) for a in (sd, md, sq, mq)]
        self.planes = [np.ascontiguousarray(a) for a in planes]
        self.rows, self.cols = rows, cols
        self.ot = OrcTensor()
        for i, a in enumerate(self.planes):
            self.ot.plane[i] = a.ctypes.data
        self.ot.sd, self.ot.md = self.arrays[0].ctypes.data, self.arrays[1].ctypes.data
        self.ot.sq, self.ot.mq = self.arrays[2].ctypes.data, self.arrays[3].ctypes.data
        self.ot.rows, self.ot.cols, self.ot.nbits, self.ot.scale6, self.ot.minneg = rows, cols, nbits, 0, 0

    def dequant(self, row):
        out = np.zeros(self.cols, np.float32)
        oracle().orc_dequant_row(ctypes.byref(self.ot), row, out.ctypes.data)
        return out

    def codes(self, row):
        out = np.zeros(self.cols, np.uint8)
        oracle().orc_unpack_row(ctypes.byref(self.ot), row, out.ctypes.data)
        return out

    def matvec(self, q, s, u):
        y = np.zeros(self.rows, np.float32)
        oracle().orc_matvec(ctypes.byref(self.ot), q.ctypes.data, s.ctypes.data, u.ctypes.data, y.ctypes.data,
                            0, self.rows)
        return y
