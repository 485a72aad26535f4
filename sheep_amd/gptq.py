"""GPTQ-style and AWQ 4-bit matrices on the device: packing, a seeded
synthetic generator and the ctypes wrapper of sml_hip_gptq_* /
sml_hip_awq_upload.

The layout is AutoGPTQ's (what tooling/sml_unpack.py:66-95 dequantizes):
rows are outputs, cols inputs; qweight int32 [cols/8, rows] with the codes of
inputs 8k..8k+7 of output o in word (k, o), input 8k+i in bits 4i..4i+3;
qzeros int32 [cols/group, rows/8] with output 8j+i's zero in bits 4i..4i+3 of
word (g, j); scales fp16 [cols/group, rows]. The v1 files store zero - 1.
"""
import ctypes

import numpy as np

from . import DevBuf, HipError, lib


def pack(codes, zeros, scales, zero_add=1):
    """codes uint8 [rows, cols] in 0..15, zeros [rows, cols/group] (the real
    zero point), scales [rows, cols/group] -> (qweight, qzeros, scales fp16)
    as stored. zero_add 1 writes the v1 form (zero - 1)."""
    codes = np.asarray(codes, np.uint32)
    rows, cols = codes.shape
    ngr = zeros.shape[1]
    c = codes.T.reshape(cols // 8, 8, rows)                    # [k, i, o]
    qweight = np.zeros((cols // 8, rows), np.uint32)
    for i in range(8):
        qweight |= c[:, i, :] << np.uint32(4 * i)
    z = (np.asarray(zeros, np.int64) - zero_add).astype(np.uint32).T.reshape(ngr, rows // 8, 8)   # [g, j, i]
    qzeros = np.zeros((ngr, rows // 8), np.uint32)
    for i in range(8):
        qzeros |= (z[:, :, i] & np.uint32(15)) << np.uint32(4 * i)
    return (qweight.view(np.int32), qzeros.view(np.int32),
            np.ascontiguousarray(np.asarray(scales, np.float16).T))


AWQ_NIBBLE = (0, 4, 1, 5, 2, 6, 3, 7)     # nibble of output 8j+k in word j (tooling/sml_unpack.py:78)


def pack_awq(codes, zeros, scales):
    """codes uint8 [rows, cols] in 0..15, zeros [rows, cols/group] (None: the
    default 8, no qzeros), scales [rows, cols/group] -> (qweight, qzeros or
    None, scales fp16) in the AWQ GEMM layout: qweight [cols, rows/8] with
    output 8j+k in nibble AWQ_NIBBLE[k] of word (input, j)."""
    codes = np.asarray(codes, np.uint32)
    rows, cols = codes.shape
    c = codes.T.reshape(cols, rows // 8, 8)                    # [k, j, i]
    qweight = np.zeros((cols, rows // 8), np.uint32)
    for i in range(8):
        qweight |= c[:, :, i] << np.uint32(4 * AWQ_NIBBLE[i])
    qzeros = None
    if zeros is not None:
        z = np.asarray(zeros, np.uint32).T.reshape(-1, rows // 8, 8)
        qzeros = np.zeros(z.shape[:2], np.uint32)
        for i in range(8):
            qzeros |= (z[:, :, i] & np.uint32(15)) << np.uint32(4 * AWQ_NIBBLE[i])
        qzeros = qzeros.view(np.int32)
    return qweight.view(np.int32), qzeros, np.ascontiguousarray(np.asarray(scales, np.float16).T)


def synth(rows, cols, seed, group=128):
    """Codes uniform over 0..15, zero point 8 (stored as 7), per-group scales
    |N(0, 0.02)| / 7 in fp16: the GPTQ-4 recipe of the width sweep."""
    rng = np.random.default_rng(seed)
    ngr = cols // group
    qweight = rng.integers(0, 1 << 32, size=(cols // 8, rows), dtype=np.uint64).astype(np.uint32).view(np.int32)
    qzeros = np.full((ngr, rows // 8), 0x77777777, np.uint32).view(np.int32)
    scales = (np.abs(rng.standard_normal((ngr, rows))) * 0.02 / 7).astype(np.float16)
    return qweight, qzeros, scales


class GptqMat:
    """A GPTQ-style matrix resident in HBM (awq=True: the arrays are in the
    AWQ layout, qzeros may be None, zero_add is ignored)."""

    def __init__(self, qweight, qzeros, scales, rows, cols, group=128, zero_add=1, awq=False, g_idx=None):
        self.rows, self.cols, self.group, self.zero_add = rows, cols, group, 0 if awq else zero_add
        qw = np.ascontiguousarray(qweight, np.int32)
        qz = None if qzeros is None else np.ascontiguousarray(qzeros, np.int32)
        sc = np.ascontiguousarray(scales, np.float16)
        if awq:
            h = lib().sml_hip_awq_upload(qw.ctypes.data, None if qz is None else qz.ctypes.data, sc.ctypes.data,
                                         rows, cols, group)
        elif g_idx is not None:
            gi = np.ascontiguousarray(g_idx, np.int32)
            h = lib().sml_hip_gptq_upload_gidx(qw.ctypes.data, qz.ctypes.data, sc.ctypes.data, gi.ctypes.data,
                                               rows, cols, group, zero_add)
        else:
            h = lib().sml_hip_gptq_upload(qw.ctypes.data, qz.ctypes.data, sc.ctypes.data, rows, cols, group,
                                          zero_add)
        if not h:
            raise HipError(f"gptq upload: {lib().sml_hip_last_error().decode(errors='replace')}")
        self.h = h
        self.bytes = lib().sml_hip_gptq_bytes(h)

    def matvec(self, x, y):
        if lib().sml_hip_gptq_matvec(self.h, x.ptr, y.ptr) != 0:
            raise HipError(f"gptq matvec: {lib().sml_hip_last_error().decode(errors='replace')}")

    def unpack(self, row0, nrows):
        c, z = DevBuf(nrows * self.cols), DevBuf(nrows * (self.cols // self.group))
        if lib().sml_hip_gptq_unpack(self.h, row0, nrows, c.ptr, z.ptr) != 0:
            raise HipError(f"gptq unpack: {lib().sml_hip_last_error().decode(errors='replace')}")
        return (c.read(np.uint8).reshape(nrows, self.cols),
                z.read(np.uint8).reshape(nrows, self.cols // self.group))

    def free(self):
        if self.h:
            lib().sml_hip_gptq_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def time_matvec(mats, x, y, iters):
    """Milliseconds for `iters` launches rotating over `mats` (HIP events)."""
    arr = (ctypes.c_void_p * len(mats))(*[m.h for m in mats])
    ms = ctypes.c_float()
    if lib().sml_hip_gptq_time(arr, len(mats), x.ptr, y.ptr, iters, ctypes.byref(ms)) != 0:
        raise HipError(f"gptq time: {lib().sml_hip_last_error().decode(errors='replace')}")
    return ms.value


def desc_act_gidx(cols, seed, group=128):
    """A desc_act g_idx: inputs taken in a random activation order, the
    order's positions grouped by `group` (g_idx[order[j]] = j // group)."""
    order = np.random.default_rng(seed).permutation(cols)
    g = np.empty(cols, np.int32)
    g[order] = np.arange(cols) // group
    return g
