"""Ingest on the GPU: GPTQ / AWQ copies re-quantized into SSF FLAT planes at a
width of their own, through libsmlhip.so.

Mirrors the reference's route for a quantized copy: tooling/sml_unpack.py
dequantizes it to float16 (dequant_gptq, dequant_awq), then the quantizer
encodes every tensor (tooling/sml_quantize.py Quantizer.run / encode /
_write). The quantizer's two fused C searches are not wrapped here: the
library exports them under the reference's own C prototypes (sml_asym_grid,
sml_field_search, sml/sml-quant.c:38-137), so the reference's loader binds
libsmlhip.so in place of its own build. Calibration (the GPTQ error feedback
and activation importance) is the reference builder's and is not part of
this path: importance weights are taken as given.
"""
import ctypes

import numpy as np

from . import DevBuf, HipError, Mat, lib

c_int, c_float, c_void_p, c_char_p = ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_char_p
_SIGS = [
    ("sml_hip_asym_grid", c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int, c_int,
                                  c_int, c_void_p, c_void_p]),
    ("sml_hip_field_search", c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                     c_int, c_int, c_int, c_void_p, c_int]),
    ("sml_asym_grid", None, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_int, c_int, c_int,
                             c_void_p, c_void_p]),
    ("sml_field_search", None, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                c_int, c_int, c_void_p, c_int]),
    ("sml_hip_unpack_dequant", c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                       c_int, c_void_p]),
    ("sml_hip_gguf_dequant", c_int, [c_int, c_void_p, c_int, c_int, c_void_p]),
    ("sml_hip_requant", c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_int, ctypes.POINTER(c_void_p),
                                c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("sml_hip_requant_last_ms", c_float, []),
    ("sml_hip_mat_from_requant", c_void_p, [ctypes.POINTER(c_void_p), c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                            c_int, c_int]),
    ("sml_hip_ssf_write_quant", c_int, [c_char_p, c_char_p, c_int, c_int, c_int, ctypes.POINTER(c_void_p), c_void_p,
                                        c_void_p, c_void_p, c_void_p, c_void_p]),
]
_bound = False

# The planes of a FLAT tensor of each width, in storage order
# (tooling/sml_quantize.py:104-106): bits per plane.
FLAT_PLANES = {2: [2], 3: [2, 1], 4: [4], 5: [4, 1], 6: [2, 4], 7: [4, 2, 1], 8: [4, 4]}
SCALE_SUPER, GROUP = 256, 32


def _lib():
    global _bound
    l = lib()
    if not _bound:
        for name, res, args in _SIGS:
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _bound = True
    return l


def _err(what):
    raise HipError(f"{what}: {lib().sml_hip_last_error().decode(errors='replace')}")


def _p(a):
    return None if a is None else a.ctypes.data


def available():
    """True when the library loads (the GPU is checked on first use)."""
    try:
        _lib()
        return True
    except (OSError, RuntimeError):
        return False


# ---------------------------------------------------------------- unpacking (tooling/sml_unpack.py)

def _dequant(qweight, qzeros, scales, g_idx, rows, cols, bits, group, zero_add, awq, out=None):
    """Device dequantization into out (DevBuf of rows*cols floats, made if None)."""
    bufs = [DevBuf.of(np.ascontiguousarray(qweight, np.int32))]
    bufs.append(DevBuf.of(np.ascontiguousarray(qzeros, np.int32)) if qzeros is not None else None)
    bufs.append(DevBuf.of(np.ascontiguousarray(scales, np.float16).view(np.uint16)))
    bufs.append(DevBuf.of(np.ascontiguousarray(g_idx, np.int32)) if g_idx is not None else None)
    out = out or DevBuf(rows * cols * 4)
    if _lib().sml_hip_unpack_dequant(bufs[0].ptr, bufs[1].ptr if bufs[1] else None, bufs[2].ptr,
                                     bufs[3].ptr if bufs[3] else None, rows, cols, bits, group, zero_add,
                                     int(awq), out.ptr) != 0:
        _err("unpack_dequant")
    return out


def _gptq_args(t, qc):
    bits = int(qc.get("bits", 4))
    qweight = np.asarray(t["qweight"])
    rows, cols = qweight.shape[1], qweight.shape[0] * (32 // bits)
    zero_add = 0 if str(qc.get("checkpoint_format") or "gptq").lower() == "gptq_v2" else 1
    g = t.get("g_idx")
    gs = int(qc.get("group_size") or -1)
    gs = cols if gs <= 0 else gs
    if g is None or not qc.get("desc_act"):
        g = None
    return (qweight, t["qzeros"], t["scales"], g, rows, cols, bits, gs, zero_add, 0)


def _awq_args(t, qc):
    bits = int(qc.get("bits", qc.get("w_bit", 4)))
    qweight = np.asarray(t["qweight"])
    per = 32 // bits
    rows, cols = qweight.shape[1] * per, qweight.shape[0]
    gs = int(qc.get("group_size", qc.get("q_group_size", 128)) or -1)
    gs = cols if gs <= 0 else gs
    return (qweight, t.get("qzeros"), t["scales"], None, rows, cols, bits, gs, 0, 1)


def dequant_gptq(t, qc):
    """GPTQ (AutoGPTQ / GPTQModel / optimum layout) to a float16 [out, in]
    weight, on the GPU. follows tooling/sml_unpack.py:84-97"""
    a = _gptq_args(t, qc)
    return _dequant(*a).read(np.float32, a[4] * a[5]).reshape(a[4], a[5]).astype(np.float16)


def dequant_awq(t, qc):
    """AWQ GEMM layout to a float16 [out, in] weight, on the GPU.
    follows tooling/sml_unpack.py:100-118"""
    a = _awq_args(t, qc)
    return _dequant(*a).read(np.float32, a[4] * a[5]).reshape(a[4], a[5]).astype(np.float16)


# ---------------------------------------------------------------- re-quantization (tooling/sml_quantize.py)

class Requantized:
    """One tensor in SSF FLAT form on the device: planes (storage order),
    sd/md [rows][cols/256] fp16, sq/mq [rows][cols/32], perm [cols], and the
    codes [rows][cols] (permuted order) when kept."""

    def __init__(self, rows, cols, nbits, keep_codes):
        self.rows, self.cols, self.nbits = rows, cols, nbits
        self.plane_bits = FLAT_PLANES[nbits]
        self.planes = [DevBuf(rows * cols * b // 8) for b in self.plane_bits]
        ng, ns = cols // GROUP, cols // SCALE_SUPER
        self.sd, self.md = DevBuf(rows * ns * 2), DevBuf(rows * ns * 2)
        self.sq, self.mq = DevBuf(rows * ng), DevBuf(rows * ng)
        self.perm = DevBuf(cols * 4)
        self.codes = DevBuf(rows * cols) if keep_codes else None
        self.ms = None

    def _pl(self):
        return (c_void_p * 3)(*([p.ptr for p in self.planes] + [None] * (3 - len(self.planes))))

    def host(self):
        """Everything fetched: dict of numpy arrays in the file's layout."""
        ng, ns = self.cols // GROUP, self.cols // SCALE_SUPER
        out = {"planes": [p.read(np.uint8).reshape(self.rows, -1) for p in self.planes],
               "sd": self.sd.read(np.uint16).reshape(self.rows, ns), "md": self.md.read(np.uint16).reshape(self.rows, ns),
               "sq": self.sq.read(np.uint8).reshape(self.rows, ng), "mq": self.mq.read(np.uint8).reshape(self.rows, ng),
               "perm": self.perm.read(np.int32)}
        if self.codes is not None:
            out["codes"] = self.codes.read(np.uint8).reshape(self.rows, self.cols)
        return out

    def mat(self):
        """The tensor as a GEMV-ready matrix."""
        return Mat(_lib().sml_hip_mat_from_requant(self._pl(), self.sd.ptr, self.sq.ptr, self.md.ptr, self.mq.ptr,
                                                   self.rows, self.cols, self.nbits))

    def write_ssf(self, path, name="w"):
        """An SSF file holding this tensor as record `name`
        (tooling/sml_quantize.py:598-651, Quantizer._write)."""
        h = self.host()
        pl = [np.ascontiguousarray(p) for p in h["planes"]]
        ptrs = (c_void_p * 3)(*([p.ctypes.data for p in pl] + [None] * (3 - len(pl))))
        if _lib().sml_hip_ssf_write_quant(str(path).encode(), name.encode(), self.rows, self.cols, self.nbits, ptrs,
                                          h["sd"].ctypes.data, h["sq"].ctypes.data, h["md"].ctypes.data,
                                          h["mq"].ctypes.data, h["perm"].ctypes.data) != 0:
            _err("ssf write")
        return path


def requantize_dev(wdev, rows, cols, nbits=4, perm=None, wt=None, radius=2, keep_codes=False):
    """Re-quantize a device float tensor [rows][cols] (DevBuf) into SSF FLAT
    width nbits. perm: column order (int32 [cols]) or None for ascending max
    |w| (the quantizer without activations, tooling/sml_quantize.py:479);
    wt: per-column weights in the permuted order, normalised, or None.
    follows tooling/sml_quantize.py:426-581 (run and encode without feedback)"""
    r = Requantized(rows, cols, nbits, keep_codes)
    pbuf = DevBuf.of(np.ascontiguousarray(perm, np.int32)) if perm is not None else None
    wbuf = DevBuf.of(np.ascontiguousarray(wt, np.float32)) if wt is not None else None
    if _lib().sml_hip_requant(wdev.ptr, rows, cols, nbits, pbuf.ptr if pbuf else None, wbuf.ptr if wbuf else None,
                              radius, r._pl(), r.sd.ptr, r.sq.ptr, r.md.ptr, r.mq.ptr, r.perm.ptr,
                              r.codes.ptr if r.codes else None) != 0:
        _err("requant")
    r.ms = _lib().sml_hip_requant_last_ms()
    return r


def requantize(w, nbits=4, perm=None, wt=None, radius=2, keep_codes=False):
    """requantize_dev for a host float array [rows][cols]."""
    w = np.ascontiguousarray(w, np.float32)
    return requantize_dev(DevBuf.of(w), w.shape[0], w.shape[1], nbits, perm, wt, radius, keep_codes)


def ingest_gptq(t, qc, nbits=None, radius=2, keep_codes=False):
    """A GPTQ tensor (dict of qweight/qzeros/scales[/g_idx]) to SSF FLAT at
    its own width (nbits None: the copy's bits), unpacked and re-quantized on
    the device without a host round trip of the float copy."""
    a = _gptq_args(t, qc)
    w = _dequant(*a)
    return requantize_dev(w, a[4], a[5], nbits or a[6], None, None, radius, keep_codes)


GGUF_TYPES = {"Q8_0": (8, 32, 34, 8), "Q4_0": (2, 32, 18, 4), "Q6_K": (14, 256, 210, 6)}   # type, weights, bytes, bits


def gguf_dequant(kind, blocks, rows, cols):
    """GGUF Q8_0 / Q4_0 / Q6_K blocks (host bytes, [rows][cols/qk][bytes]) to
    the float16 copy in fp32 on the device (sml_hip_gguf_dequant)."""
    gtype, qk, bs, _ = GGUF_TYPES[kind]
    raw = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    if cols % qk or raw.size != rows * (cols // qk) * bs:
        raise ValueError(f"{kind} {rows}x{cols}: {raw.size} bytes is not whole blocks")
    src = DevBuf.of(raw)
    out = DevBuf(rows * cols * 4)
    if _lib().sml_hip_gguf_dequant(gtype, src.ptr, rows, cols, out.ptr) != 0:
        _err("gguf_dequant")
    return out


def ingest_gguf(kind, blocks, rows, cols, nbits=None, radius=2, keep_codes=False):
    """A GGUF Q8_0 / Q4_0 / Q6_K tensor to SSF FLAT (nbits None: the block
    type's own width), dequantized and re-quantized on the device, the route
    the reference takes for a GGUF it reads through transformers."""
    w = gguf_dequant(kind, blocks, rows, cols)
    return requantize_dev(w, rows, cols, nbits or GGUF_TYPES[kind][3], None, None, radius, keep_codes)


def ingest_awq(t, qc, nbits=None, radius=2, keep_codes=False):
    """An AWQ tensor to SSF FLAT at its own width, as ingest_gptq."""
    a = _awq_args(t, qc)
    w = _dequant(*a)
    return requantize_dev(w, a[4], a[5], nbits or a[6], None, None, radius, keep_codes)


def pack_gptq(codes, zeros, scales, bits, zero_add=1):
    """codes [rows, cols] (0..2^bits-1), zeros [rows, groups] (the real zero
    point), scales [rows, groups] -> (qweight, qzeros, scales fp16) in the
    GPTQ layout of `bits` (2, 4 or 8), v1 (zero - 1) for zero_add 1: the
    inverse of tooling/sml_unpack.py:66-76,84-89."""
    per = 32 // bits
    codes = np.asarray(codes, np.uint32)
    rows, cols = codes.shape
    ngr = zeros.shape[1]
    c = codes.T.reshape(cols // per, per, rows)
    qweight = np.zeros((cols // per, rows), np.uint32)
    for i in range(per):
        qweight |= c[:, i, :] << np.uint32(bits * i)
    mask = np.uint32((1 << bits) - 1)
    z = (np.asarray(zeros, np.int64) - zero_add).astype(np.uint32).T.reshape(ngr, rows // per, per)
    qzeros = np.zeros((ngr, rows // per), np.uint32)
    for i in range(per):
        qzeros |= (z[:, :, i] & mask) << np.uint32(bits * i)
    return qweight.view(np.int32), qzeros.view(np.int32), np.ascontiguousarray(np.asarray(scales, np.float16).T)
