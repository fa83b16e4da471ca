"""Restatement of the FLKV bundle codec and of the cache's prefix export / import gather.

TEST INFRASTRUCTURE ONLY: used by tests/ and bench.py's CPU baseline as the checker of the
library's bundle export / import; never by the product path (flour_amd/).

Follows (reference files, lltsdyp/flour):
  src/kv_cache/bundle.rs:1-22     the frame: "FLKV", version u16 LE, header_len u32 LE, the
                                  KvBundleMeta JSON header, then per logical block, per layer, the
                                  K block and the V block, (num_kv_heads, block_size, head_dim)
  src/kv_cache/bundle.rs:71-81    KvBundleMeta fields, in declaration order (serde's order)
  src/kv_cache/bundle.rs:108-143  KvBundleCodec::encode (serde_json::to_vec: compact)
  src/kv_cache/bundle.rs:145-214  KvBundleCodec::decode and its checks
  src/models/common/cache.rs:166-229  export_prefix_bundle: logical block b reads the pool run
                                  starting at slot(b * block_size) of every layer
The header is written with Python's json module (compact separators, non-ASCII verbatim),
which escapes strings as serde_json does; tests pin that against hand-made frames.
"""
from __future__ import annotations

import json
import struct

import numpy as np

MAGIC = b"FLKV"
VERSION = 1
DTYPE_BYTES = {"F32": 4, "F16": 2, "BF16": 2}
FIELDS = ("model_id", "token_count", "token_ids", "block_size", "num_layers", "num_kv_heads",
          "head_dim", "dtype")


class BundleError(ValueError):
    pass


def header_json(meta: dict) -> bytes:
    """KvBundleMeta as serde_json::to_vec writes it (fields in declaration order)."""
    ordered = {k: meta[k] for k in FIELDS}
    return json.dumps(ordered, separators=(",", ":"), ensure_ascii=False).encode("utf-8")


def encode(meta: dict, blocks: list[list[tuple[np.ndarray, np.ndarray]]]) -> bytes:
    """KvBundleCodec::encode: blocks[b][layer] = (k, v), each (num_kv_heads, block_size,
    head_dim) arrays whose raw bytes are the element type's little-endian encoding."""
    bs = meta["block_size"]
    if bs == 0 or meta["token_count"] % bs:
        raise BundleError(f"bundle token_count {meta['token_count']} not block aligned")
    if len(blocks) != meta["token_count"] // bs:
        raise BundleError("bundle block count")
    hdr = header_json(meta)
    out = [MAGIC, struct.pack("<H", VERSION), struct.pack("<I", len(hdr)), hdr]
    for layers in blocks:
        if len(layers) != meta["num_layers"]:
            raise BundleError("block layer count")
        for k, v in layers:
            out.append(np.ascontiguousarray(k).tobytes())
            out.append(np.ascontiguousarray(v).tobytes())
    return b"".join(out)


def decode(data: bytes, np_dtype) -> tuple[dict, list[list[tuple[np.ndarray, np.ndarray]]]]:
    """KvBundleCodec::decode, with its checks in its order. ``np_dtype`` is the numpy type that
    holds one element (float32, or uint16 for the 16-bit types)."""
    if len(data) < 10:
        raise BundleError(f"bundle too short: {len(data)} bytes")
    if data[:4] != MAGIC:
        raise BundleError("bad bundle magic")
    (version,) = struct.unpack("<H", data[4:6])
    if version != VERSION:
        raise BundleError(f"unsupported bundle version {version}")
    (hl,) = struct.unpack("<I", data[6:10])
    if len(data) < 10 + hl:
        raise BundleError("bundle header truncated")
    meta = json.loads(data[10:10 + hl].decode("utf-8"))
    for f in FIELDS:
        if f not in meta:
            raise BundleError(f"missing field `{f}`")
    if meta["block_size"] == 0:
        raise BundleError("bundle block_size is zero")
    if meta["token_count"] == 0 or meta["token_count"] % meta["block_size"]:
        raise BundleError("bundle token_count not block aligned")
    if len(meta["token_ids"]) != meta["token_count"]:
        raise BundleError("bundle token_ids len != token_count")
    nb = meta["token_count"] // meta["block_size"]
    shape = (meta["num_kv_heads"], meta["block_size"], meta["head_dim"])
    per = int(np.prod(shape)) * DTYPE_BYTES[meta["dtype"]]
    payload = data[10 + hl:]
    if len(payload) != nb * meta["num_layers"] * 2 * per:
        raise BundleError("bundle payload length")
    blocks, off = [], 0
    for _ in range(nb):
        layers = []
        for _ in range(meta["num_layers"]):
            k = np.frombuffer(payload[off:off + per], dtype=np_dtype).reshape(shape)
            v = np.frombuffer(payload[off + per:off + 2 * per], dtype=np_dtype).reshape(shape)
            layers.append((k, v))
            off += 2 * per
        blocks.append(layers)
    return meta, blocks


def gather_blocks(k_pools: list[np.ndarray], v_pools: list[np.ndarray], block_ids, block_size: int,
                  num_blocks: int) -> list[list[tuple[np.ndarray, np.ndarray]]]:
    """export_prefix_bundle's read: logical block b of every layer is the pool run of block_size
    slots starting at block_ids[b] * block_size (slot(b * bs), cache.rs:205-209), for all heads.
    Pools are host copies (kv_heads, num_slots, head_dim)."""
    out = []
    for b in range(num_blocks):
        s0 = int(block_ids[b]) * block_size
        out.append([(k[:, s0:s0 + block_size].copy(), v[:, s0:s0 + block_size].copy())
                    for k, v in zip(k_pools, v_pools)])
    return out


def export_frame(model_id: str, token_ids, token_count: int, k_pools, v_pools, block_ids,
                 block_size: int, dtype: str) -> bytes:
    """The frame export_prefix_bundle + encode produce for a cache whose live table is
    ``block_ids`` (host pool copies per layer)."""
    G, _, D = k_pools[0].shape
    meta = {"model_id": model_id, "token_count": token_count,
            "token_ids": [int(t) for t in token_ids[:token_count]], "block_size": block_size,
            "num_layers": len(k_pools), "num_kv_heads": G, "head_dim": D, "dtype": dtype}
    return encode(meta, gather_blocks(k_pools, v_pools, block_ids, block_size,
                                      token_count // block_size))
