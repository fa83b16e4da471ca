"""FLKV bundle frame (src/kv_cache/bundle.rs) on the CPU: the oracle's codec against the
reference's own codec tests, layout pins fixed by the format description, and the library's
frame decoding and validation (flour_kv_cache_import_bundle on a bookkeeping-only cache, which
reaches "no device pool" only after every check of decode and import_prefix_bundle passed).

Pins: the reference tests bundle.rs:279-417 (sample bundle round trip; corrupt magic, unknown
version, wrong payload length, truncated header rejected; f16 bits preserved); the byte layout
of bundle.rs:7-22 (magic, little-endian version and header length, block -> layer -> K, V
payload order) read back from fixed offsets; serde_json's compact output and string escapes
(quote, backslash, \\b \\f \\n \\r \\t, \\u00xx for other control characters, the rest verbatim)
checked on a hand-written header.
"""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest

import flkv as F
from flour_amd import _lib
from flour_amd.kv_cache import KvCache


def sample_bundle():
    """bundle.rs:279-319: 2 blocks, 2 layers, kv_heads 1, block_size 2, head_dim 2, F32,
    K = base + i with base = b * 100 + l * 10, V = K + 0.5."""
    blocks = []
    for b in range(2):
        layers = []
        for l in range(2):
            k = (b * 100 + l * 10 + np.arange(4, dtype=np.float32)).reshape(1, 2, 2)
            layers.append((k, k + np.float32(0.5)))
        blocks.append(layers)
    meta = {"model_id": "model-a", "token_count": 4, "token_ids": [0, 1, 2, 3], "block_size": 2,
            "num_layers": 2, "num_kv_heads": 1, "head_dim": 2, "dtype": "F32"}
    return meta, blocks


def test_reference_round_trip_bundle_rs_328():
    meta, blocks = sample_bundle()
    data = F.encode(meta, blocks)
    m2, b2 = F.decode(data, np.float32)
    assert m2 == meta
    for (k1, v1), (k2, v2) in zip([x for l in blocks for x in l], [x for l in b2 for x in l]):
        assert np.array_equal(k1, k2) and np.array_equal(v1, v2)


@pytest.mark.parametrize("mutate,what", [
    (lambda d: b"X" + d[1:], "bad bundle magic"),                       # bundle.rs:345
    (lambda d: d[:4] + bytes([9, 0]) + d[6:], "unsupported bundle version 9"),  # :352
    (lambda d: d[:-1], "bundle payload length"),                        # :361
    (lambda d: d[:8], "bundle too short"),                              # :369 (prefix cut)
])
def test_reference_rejections(mutate, what):
    meta, blocks = sample_bundle()
    with pytest.raises(F.BundleError, match=what.split(" 9")[0]):
        F.decode(mutate(F.encode(meta, blocks)), np.float32)


def test_f16_bits_round_trip_bundle_rs_378():
    k = np.array([1.5, -2.0], np.float16).view(np.uint16).reshape(1, 2, 1)
    meta = {"model_id": "m", "token_count": 2, "token_ids": [0, 1], "block_size": 2,
            "num_layers": 1, "num_kv_heads": 1, "head_dim": 1, "dtype": "F16"}
    _, blocks = F.decode(F.encode(meta, [[(k, k)]]), np.uint16)
    assert np.array_equal(blocks[0][0][0].view(np.float16).ravel(), np.array([1.5, -2.0], np.float16))


def test_layout_read_back_at_fixed_offsets():
    meta, blocks = sample_bundle()
    data = F.encode(meta, blocks)
    assert data[:4] == b"FLKV" and struct.unpack("<H", data[4:6])[0] == 1
    (hl,) = struct.unpack("<I", data[6:10])
    hdr = data[10:10 + hl]
    assert hdr == (b'{"model_id":"model-a","token_count":4,"token_ids":[0,1,2,3],"block_size":2,'
                   b'"num_layers":2,"num_kv_heads":1,"head_dim":2,"dtype":"F32"}')
    pay = np.frombuffer(data[10 + hl:], np.float32)
    assert pay.size == 2 * 2 * 2 * 4
    # block 1, layer 0: K at (1 * 2 + 0) * 2 tensors in, V right after it
    assert list(pay[16:20]) == [100, 101, 102, 103] and list(pay[20:24]) == [100.5, 101.5, 102.5, 103.5]
    assert list(pay[4:8]) == [0.5, 1.5, 2.5, 3.5]            # block 0 layer 0 V
    assert list(pay[8:12]) == [10, 11, 12, 13]               # block 0 layer 1 K


def test_header_escapes_follow_serde_json():
    meta, _ = sample_bundle()
    meta = dict(meta, model_id='a"b\\c\n\t\x01\x1f\x7f/é')
    hdr = F.header_json(meta)
    assert hdr.startswith('{"model_id":"a\\"b\\\\c\\n\\t\\u0001\\u001f\x7f/é",'.encode("utf-8"))


# ------------------------------------------------------------------ the library's decoder

def frame(meta: dict, payload_bytes: int | None = None, header: bytes | None = None) -> bytes:
    hdr = F.header_json(meta) if header is None else header
    n = payload_bytes
    if n is None:
        nb = meta["token_count"] // meta["block_size"]
        n = nb * meta["num_layers"] * 2 * meta["num_kv_heads"] * meta["block_size"] * \
            meta["head_dim"] * F.DTYPE_BYTES[meta["dtype"]]
    return b"FLKV" + struct.pack("<HI", 1, len(hdr)) + hdr + bytes(n)


def cache_meta(**kw):
    m = {"model_id": "m", "token_count": 32, "token_ids": list(range(32)), "block_size": 16,
         "num_layers": 2, "num_kv_heads": 2, "head_dim": 4, "dtype": "F32"}
    m.update(kw)
    return m


@pytest.fixture
def host_cache():
    import torch
    return KvCache(2, 64, 2, 2, 4, torch.float32, 16, device_pool=False)


def import_error(cache, data, prompt=range(40)) -> str:
    with pytest.raises(_lib.FlourError) as e:
        cache.import_prefix_bundle(data, list(prompt))
    return str(e.value)


def test_valid_frames_pass_every_check(host_cache):
    # every check of decode + import_prefix_bundle passes; only the device copy is missing
    assert "no device pool" in import_error(host_cache, frame(cache_meta()))
    # any field order, whitespace and unknown fields, as serde_json accepts them
    m = cache_meta()
    hdr = (' {\n "dtype" : "F32", "head_dim":4, "extra": {"a": [1, -2.5e3, null, true]}, '
           '"num_kv_heads":2,"num_layers":2,"block_size":16,"token_ids":' + json.dumps(m["token_ids"]) +
           ',"token_count":32,"model_id":"\\u006d"}\t').encode()
    assert "no device pool" in import_error(host_cache, frame(m, header=hdr))


@pytest.mark.parametrize("edit,what", [
    (lambda m: (m, None, b'{"model_id":"m"}'), "missing field `token_count`"),
    (lambda m: (m, None, F.header_json(m)[:-1] + b',"head_dim":4}'), "duplicate field `head_dim`"),
    (lambda m: (m, None, F.header_json(m).replace(b'"head_dim":4', b'"head_dim":-4')), "invalid value"),
    (lambda m: (m, None, F.header_json(m).replace(b'"head_dim":4', b'"head_dim":4.0')), "floating point"),
    (lambda m: (m, None, F.header_json(m).replace(b'[0,', b'[4294967296,')), "expected u32"),
    (lambda m: (m, None, F.header_json(m).replace(b'"F32"', b'"F64"')), "unknown variant `F64`"),
    (lambda m: (m, None, F.header_json(m).replace(b'"m"', b'"\\x"')), "invalid escape"),
    (lambda m: (m, None, F.header_json(m).replace(b'"m"', b'"\\ud800"')), "hex escape"),
    (lambda m: (m, None, F.header_json(m).replace(b'"m"', b'"a\nb"')), "control character"),
    (lambda m: (m, None, F.header_json(m) + b" x"), "trailing characters"),
    (lambda m: (dict(m, block_size=0), 0, None), "bundle block_size is zero"),
    (lambda m: (dict(m, token_count=20, token_ids=list(range(20))), 0, None), "not block aligned"),
    (lambda m: (dict(m, token_ids=list(range(31))), None, None), "token_ids len 31 != token_count 32"),
    (lambda m: (m, 7, None), "bundle payload length 7 != expected"),
    (lambda m: (dict(m, block_size=8, token_ids=list(range(32))), None, None), "bundle block_size 8 != cache block_size 16"),
    (lambda m: (dict(m, num_layers=3), None, None), "bundle num_layers 3 != model 2"),
    (lambda m: (dict(m, num_kv_heads=1), None, None), "bundle num_kv_heads 1 != model 2"),
    (lambda m: (dict(m, head_dim=8), None, None), "bundle head_dim 8 != model 4"),
    (lambda m: (dict(m, dtype="BF16"), None, None), "bundle dtype BF16 != model dtype"),
])
def test_rejections(host_cache, edit, what):
    m, n, hdr = edit(cache_meta())
    assert what in import_error(host_cache, frame(m, n, hdr))


def test_prefix_and_frame_rejections(host_cache):
    good = frame(cache_meta())
    assert "prompt does not start with bundle token ids" in import_error(host_cache, good, range(100, 140))
    assert "prompt does not start" in import_error(host_cache, good, range(31))
    assert "bundle too short: 3 bytes" in import_error(host_cache, b"FLK")
    assert "bad bundle magic" in import_error(host_cache, b"XLKV" + good[4:])
    assert "unsupported bundle version 2" in import_error(host_cache, good[:4] + b"\x02\x00" + good[6:])
    assert "bundle header truncated" in import_error(host_cache, good[:12])
    # a rejected import leaves the cache as it was
    assert host_cache.len() == 0 and host_cache.free_blocks() == 4


def test_export_size_and_validation(host_cache):
    import ctypes

    from flour_amd._lib import lib

    host_cache.allocate_kv(32)
    ids = np.arange(32, dtype=np.uint32)
    size = ctypes.c_size_t(0)
    rc = lib().flour_kv_cache_export_bundle(host_cache._h, b"m", ids.ctypes.data_as(ctypes.c_void_p),
                                            32, 32, None, 0, ctypes.byref(size), None)
    assert rc == 0
    k = [np.zeros((2, 64, 4), np.float32)] * 2
    want = F.export_frame("m", ids, 32, k, k, [0, 1], 16, "F32")
    assert size.value == len(want)
    for n, what in [(20, "export token_count 20 not aligned to block size 16"),
                    (48, "export token_count 48 exceeds live len 32")]:
        rc = lib().flour_kv_cache_export_bundle(host_cache._h, b"m", ids.ctypes.data_as(ctypes.c_void_p),
                                                32, n, None, 0, ctypes.byref(size), None)
        assert rc == _lib.ERR_INVALID_ARGUMENT and lib().flour_hip_last_error().decode() == what
    rc = lib().flour_kv_cache_export_bundle(host_cache._h, b"m", ids.ctypes.data_as(ctypes.c_void_p),
                                            16, 32, None, 0, ctypes.byref(size), None)
    assert lib().flour_hip_last_error().decode() == "token_ids len 16 shorter than token_count 32"
