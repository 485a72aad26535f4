"""A read-only numpy view of an SSF file.

An independent reading of the on-disk layout (the packed header and tensor
record of sml/sml-model.h:78-160, the FLAT planes of tooling/sml_quantize.py:
598-651), used by the tests to hand the same bytes to the GPU library, the
oracle and the reference build.
"""
import struct

import numpy as np

HEADER_FMT = "<4sI7I2f2I4IQ6Q2I2f2I2I3f2I2ff2I3I2ff2I"
REC_FMT = "<64s4I2Q2Q2Q2Q2Q2Q4Q4Q2I"
HEADER_FIELDS = ("magic version n_layer n_embd n_head n_head_kv n_ff n_vocab n_ctx_train rope_theta rms_eps "
                 "group n_levels lb0 lb1 lb2 lb3 n_tensors table_off json_off json_n tok_off tok_n group_off "
                 "norm_type rope_type attn_scale logit_softcap n_swa arch_bits n_rot flags emb_scale res_scale "
                 "logit_scale n_expert_used moe_flags attn_softcap clip_qkv moe_scale moe_groups moe_topk_group "
                 "ssm_groups ssm_dstate ssm_norm_group ssm_dt_lo ssm_dt_hi ssm_bcdt_eps gdn_nk gdn_dk").split()
REC_FIELDS = ("name kind rows cols group f32_off f32_bytes sd_off sd_bytes sq_off sq_bytes perm_off perm_bytes "
              "md_off md_bytes mq_off mq_bytes p0 p1 p2 p3 n0 n1 n2 n3 layout nbits").split()
HEADER_SIZE = struct.calcsize(HEADER_FMT)
REC_SIZE = struct.calcsize(REC_FMT)
# plane widths of a FLAT record per code width, in storage order
FLAT_PLANES = {2: [2], 3: [2, 1], 4: [4], 5: [4, 1], 6: [2, 4], 7: [4, 2, 1], 8: [4, 4]}


class Tensor:
    def __init__(self, f, rec):
        self.f = f
        self.rec = rec
        self.name = rec["name"]
        self.rows, self.cols = rec["rows"], rec["cols"]
        self.nbits = rec["nbits"]

    def _arr(self, off, n, dtype):
        return np.frombuffer(self.f.mm, dtype=dtype, count=n, offset=off)

    @property
    def f32(self):
        return self._arr(self.rec["f32_off"], self.rows * self.cols, np.float32)

    def plane(self, i):
        return self._arr(self.rec[f"p{i}"], self.rec[f"n{i}"], np.uint8)

    def planes(self):
        return [self.plane(i) for i in range(len(FLAT_PLANES[self.nbits]))]

    @property
    def perm(self):
        return self._arr(self.rec["perm_off"], self.cols, np.int32)

    @property
    def sd(self):
        return self._arr(self.rec["sd_off"], self.rec["sd_bytes"] // 2, np.uint16)

    @property
    def sq(self):
        return self._arr(self.rec["sq_off"], self.rec["sq_bytes"], np.uint8)

    @property
    def md(self):
        return self._arr(self.rec["md_off"], self.rec["md_bytes"] // 2, np.uint16) if self.rec["mq_bytes"] else None

    @property
    def mq(self):
        return self._arr(self.rec["mq_off"], self.rec["mq_bytes"], np.uint8) if self.rec["mq_bytes"] else None

    def nbytes(self):
        """Codes and fields: what one pass over the matrix reads."""
        r = self.rec
        return sum(r[f"n{i}"] for i in range(4)) + r["sd_bytes"] + r["sq_bytes"] + r["md_bytes"] + r["mq_bytes"]


class SSF:
    def __init__(self, path):
        self.path = str(path)
        self.mm = np.memmap(self.path, dtype=np.uint8, mode="r")
        vals = struct.unpack_from(HEADER_FMT, self.mm, 0)
        self.hdr = dict(zip(HEADER_FIELDS, vals))
        if self.hdr["magic"] != b"SSF ":
            raise ValueError(f"{path}: not an SSF file")
        self.tensors = {}
        off = self.hdr["table_off"]
        for i in range(self.hdr["n_tensors"]):
            rec = dict(zip(REC_FIELDS, struct.unpack_from(REC_FMT, self.mm, off + i * REC_SIZE)))
            rec["name"] = rec["name"].split(b"\0", 1)[0].decode()
            self.tensors[rec["name"]] = Tensor(self, rec)

    def __getitem__(self, name):
        return self.tensors[name]

    def __contains__(self, name):
        return name in self.tensors
