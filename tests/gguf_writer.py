"""Minimal GGUF v3 writer for malformed-file tests (test helper, host only).

Builds a tiny Llama-architecture image (gguf/mod.rs:161-230 container,
llama.rs:1038-1090 keys and tensor names) from a list of tensor records that a
test may edit before serialising: shapes, types, offsets and metadata can be
made inconsistent on purpose. Tensor payloads are random bytes; only the
layout matters to the reader.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

BLOCK = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


@dataclass
class T:
    name: str
    ne: list
    type: int
    off: int | None = None  # None: packed after the previous tensor
    payload: int | None = None  # bytes to emit (None: what the shape needs)


@dataclass
class Image:
    meta: list = field(default_factory=list)  # (key, gguf value type, value)
    tensors: list = field(default_factory=list)
    version: int = 3
    align: int = 32
    n_tensors: int | None = None  # override the declared counts
    n_kv: int | None = None

    def tensor(self, name):
        return next(t for t in self.tensors if t.name == name)

    def set_meta(self, key, vt, value):
        self.meta = [m for m in self.meta if m[0] != key] + [(key, vt, value)]

    def to_bytes(self, seed: int = 0) -> bytes:
        rng = np.random.default_rng(seed)
        out = bytearray(b"GGUF")
        out += struct.pack("<I", self.version)
        out += struct.pack("<QQ", len(self.tensors) if self.n_tensors is None else self.n_tensors,
                           len(self.meta) if self.n_kv is None else self.n_kv)
        for key, vt, value in self.meta:
            kb = key.encode()
            out += struct.pack("<Q", len(kb)) + kb + struct.pack("<I", vt)
            if vt == 4:
                out += struct.pack("<I", value)
            elif vt == 6:
                out += struct.pack("<f", value)
            elif vt == 8:
                vb = value.encode()
                out += struct.pack("<Q", len(vb)) + vb
            elif vt == 9:  # array of u32
                out += struct.pack("<IQ", 4, len(value)) + b"".join(struct.pack("<I", v) for v in value)
            elif vt == 10:
                out += struct.pack("<Q", value)
            else:
                raise ValueError(vt)
        offs, cur = [], 0
        for t in self.tensors:
            n = int(np.prod(t.ne, dtype=np.uint64)) if all(x < 2**32 for x in t.ne) else 0
            be, bb = BLOCK.get(t.type, (1, 1))
            size = t.payload if t.payload is not None else n // be * bb
            off = cur if t.off is None else t.off
            offs.append((off, size))
            cur = max(cur, (off + size + self.align - 1) // self.align * self.align) if t.off is None else cur
        for t, (off, _) in zip(self.tensors, offs):
            nb = t.name.encode()
            out += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(t.ne))
            out += b"".join(struct.pack("<Q", x) for x in t.ne)
            out += struct.pack("<IQ", t.type, off)
        pad = (-len(out)) % self.align
        out += bytes(pad)
        end = 0
        for off, size in offs:
            if off < 2**40:
                end = max(end, off + size)
        out += rng.integers(0, 256, size=end, dtype=np.uint8).tobytes()
        return bytes(out)


def tiny_llama(n_layer=1, d=256, n_head=4, n_kv=2, ff=512, V=64, wtype=8) -> Image:
    """A valid tiny Llama image: Q8_0 (or Q4_K) matrices, f32 norms."""
    img = Image()
    img.meta = [("general.architecture", 8, "llama"), ("llama.block_count", 4, n_layer),
                ("llama.attention.head_count", 4, n_head), ("llama.attention.head_count_kv", 4, n_kv),
                ("llama.embedding_length", 4, d), ("llama.feed_forward_length", 4, ff),
                ("llama.context_length", 4, 1024), ("llama.rope.freq_base", 6, 10000.0),
                ("llama.attention.layer_norm_rms_epsilon", 6, 1e-5), ("general.alignment", 4, 32)]
    hd = d // n_head
    dkv = hd * n_kv
    img.tensors = [T("token_embd.weight", [d, V], wtype), T("output_norm.weight", [d], 0),
                   T("output.weight", [d, V], wtype)]
    for l in range(n_layer):
        b = f"blk.{l}."
        img.tensors += [T(b + "attn_norm.weight", [d], 0), T(b + "ffn_norm.weight", [d], 0),
                        T(b + "attn_q.weight", [d, d], wtype), T(b + "attn_k.weight", [d, dkv], wtype),
                        T(b + "attn_v.weight", [d, dkv], wtype), T(b + "attn_output.weight", [d, d], wtype),
                        T(b + "ffn_gate.weight", [d, ff], wtype), T(b + "ffn_up.weight", [d, ff], wtype),
                        T(b + "ffn_down.weight", [ff, d], wtype)]
    return img
