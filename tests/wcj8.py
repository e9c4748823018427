"""A pure-Python reader/writer of the WCJ8 job bytes, for tests.

Independent of the C++ codec it cross-checks. The section order, widths and
count prefixes restate the reference's writer and reader
(engine/src/serialize.rs:1052-1129 and 1131-1261): little-endian u32 magic
"WCJ8" and version 8, the run metadata, four header counts, then every array
as a u32 element count followed by its elements (u8, u32 or f32), then the
root beliefs and the carried roots.
"""
from __future__ import annotations

import struct

import numpy as np

MAGIC = 0x57434A38
VERSION = 8

# (name, kind) in byte order after the header counts.
TABLE_FIELDS = [
    ("node_kind", "u8"), ("node_player", "u8"),
    ("node_child_start", "u32"), ("node_child", "u32"),
    ("obs_off", "u32"), ("obs_start", "u32"), ("obs_act", "u32"), ("obs_child", "u32"),
    ("legal_row_of", "u32"), ("legal_off", "u32"), ("legal_action", "u32"), ("legal_child", "u32"),
    ("legal_trans", "u32"), ("cell_row", "u32"),
    ("draw_off", "u32"), ("draw_to", "u32"), ("draw_p", "f32"), ("draw_row_off", "u32"),
    ("draw_row_start", "u32"),
    ("cfg_off", "u32"), ("reach_off", "u32"), ("soff", "u32"), ("node_parent", "u32"),
    ("rev_row_of", "u32"), ("rev_start", "u32"), ("rev_src", "u32"), ("rev_cell", "u32"),
    ("rvd_row_of", "u32"), ("rvd_start", "u32"), ("rvd_src", "u32"), ("rvd_p", "f32"),
    ("leaf_rows", "u32"), ("term_leaves", "u32"), ("terminal_utility", "f32"),
    ("leaf_coff", "u32"), ("leaf_cidx", "u32"), ("snap_coff", "u32"),
    ("leaf_raw", "u8"), ("card_feat", "f32"),
    ("cphi", "f32"), ("cplayer", "u8"),
    ("bfs_order", "u32"), ("level_start", "u32"),
]
NONE = 0xFFFFFFFF
_NP = {"u8": np.uint8, "u32": np.uint32, "f32": np.float32}


class _Reader:
    def __init__(self, b: bytes):
        self.b = b
        self.at = 0

    def take(self, n):
        if n > len(self.b) - self.at:
            raise ValueError("truncated")
        out = self.b[self.at:self.at + n]
        self.at += n
        return out

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def f32(self):
        return struct.unpack("<f", self.take(4))[0]

    def arr(self, kind):
        n = self.u32()
        width = 1 if kind == "u8" else 4
        return np.frombuffer(self.take(n * width), dtype=np.dtype(_NP[kind]).newbyteorder("<")).astype(_NP[kind])


def decode(b: bytes) -> dict:
    r = _Reader(b)
    if r.u32() != MAGIC:
        raise ValueError("bad magic")
    if r.u32() != VERSION:
        raise ValueError("bad version")
    job = {"depth": r.u32(), "iters": r.u32(), "snapshots": r.take(1)[0] != 0}
    job["alpha"], job["beta"], job["gamma"], job["predict"] = (r.f32() for _ in range(4))
    job["snap_iters"] = r.arr("u32")
    job["net_dims"] = r.arr("u32")
    for k in ("nodes", "ncfg", "rows", "ncells"):
        job[k] = r.u32()
    for name, kind in TABLE_FIELDS:
        job[name] = r.arr(kind)
    job["root"] = [r.arr("f32"), r.arr("f32")]
    job["carried"] = [[r.arr("f32"), r.arr("f32")] for _ in range(r.u32())]
    if r.at != len(b):
        raise ValueError("trailing bytes")
    return job


def encode(job: dict) -> bytes:
    out = [struct.pack("<II", MAGIC, VERSION), struct.pack("<II", job["depth"], job["iters"]),
           bytes([1 if job["snapshots"] else 0]),
           struct.pack("<ffff", job["alpha"], job["beta"], job["gamma"], job["predict"])]

    def arr(a, kind):
        a = np.ascontiguousarray(a, dtype=_NP[kind])
        return struct.pack("<I", a.size) + a.astype(np.dtype(_NP[kind]).newbyteorder("<")).tobytes()

    out.append(arr(job["snap_iters"], "u32"))
    out.append(arr(job["net_dims"], "u32"))
    out.append(struct.pack("<IIII", job["nodes"], job["ncfg"], job["rows"], job["ncells"]))
    for name, kind in TABLE_FIELDS:
        out.append(arr(job.get(name, []), kind))
    out.append(arr(job["root"][0], "f32"))
    out.append(arr(job["root"][1], "f32"))
    out.append(struct.pack("<I", len(job["carried"])))
    for a, b in job["carried"]:
        out.append(arr(a, "f32"))
        out.append(arr(b, "f32"))
    return b"".join(out)


def mlp_payload(net_dims, rows, ncfg):
    """Widths of the network-row payload for a synthetic MLP tag
    [101, in, hidden, layers, heads, pool]: leaf_raw bytes per row, cphi floats."""
    _, inp, _, _, _, pool = [int(x) for x in net_dims]
    return rows * (inp - 2 * pool - 1), ncfg * (1 + pool)
