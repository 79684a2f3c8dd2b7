"""Weights from .safetensors files (src/safetensor.pas:466-513, 584-683).

CPU tests: the header reader against the committed byte-built fixture, against
an independent reader (the `safetensors` package), and its error handling.
GPU tests: a weight loaded from the file multiplies exactly like the same
array uploaded directly, for BF16, F32 (ties to even or truncated like the
reference's SingleToBF16) and F16, and a sharded checkpoint resolves through
its index.
"""
import json
import os
import shutil

import numpy as np
import pytest

import oracle
from invision_amd import hip
from invision_amd import quicknn_hip as q
from invision_amd.bf16 import as_bf16_bits

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIX = os.path.join(GOLD, "linear_tiny.safetensors")
EXP = np.load(os.path.join(GOLD, "linear_tiny_expected.npz"))
N, K = 12, 24


def header(path):
    raw = open(path, "rb").read()
    h = int.from_bytes(raw[:8], "little")
    return json.loads(raw[8:8 + h]), 8 + h, raw


# ---------------------------------------------------------------- CPU: header --

def test_info_matches_fixture():
    hdr, base, _ = header(FIX)
    for name, off in zip(EXP["names"], EXP["data_offsets"]):
        info = q.safetensors_info(FIX, str(name))
        assert info["dtype"] == hdr[name]["dtype"]
        assert info["shape"] == tuple(hdr[name]["shape"])
        assert info["data_offset"] == int(off) == base + hdr[name]["data_offsets"][0]


def test_info_bytes_agree_with_independent_reader():
    """The offsets we report select the same bytes the safetensors package decodes."""
    st = pytest.importorskip("safetensors")
    torch = pytest.importorskip("torch")
    raw = open(FIX, "rb").read()
    with st.safe_open(FIX, framework="pt") as f:
        assert sorted(f.keys()) == sorted(str(n) for n in EXP["names"])
        for name in f.keys():
            t = f.get_tensor(name)
            info = q.safetensors_info(FIX, name)
            nbytes = t.numel() * t.element_size()
            ours = raw[info["data_offset"]:info["data_offset"] + nbytes]
            theirs = t.contiguous().view(torch.uint8).numpy().tobytes()
            assert ours == theirs, name
            assert info["shape"] == tuple(t.shape)


def test_fixture_values():
    raw = open(FIX, "rb").read()
    info = q.safetensors_info(FIX, "blocks.0.attn.qkv.weight")
    w = np.frombuffer(raw, "<u2", N * K, info["data_offset"]).reshape(N, K)
    np.testing.assert_array_equal(w, EXP["w_bf16"])
    info = q.safetensors_info(FIX, "blocks.0.mlp.fc32.weight")
    w = np.frombuffer(raw, "<f4", N * K, info["data_offset"]).reshape(N, K)
    np.testing.assert_array_equal(w.view(np.uint32), EXP["w32"].view(np.uint32))


def _error(fn, *args):
    with pytest.raises(hip.HipError) as e:
        fn(*args)
    return str(e.value)


def test_missing_file_and_tensor():
    assert "cannot open" in _error(q.safetensors_info, "/nonexistent/x.safetensors", "w")
    assert "no tensor" in _error(q.safetensors_info, FIX, "blocks.9.missing")
    assert "no tensor" in _error(q.safetensors_info, FIX, "__metadata__")  # metadata is not a tensor


def _write(tmp_path, name, data):
    p = os.path.join(tmp_path, name)
    with open(p, "wb") as f:
        f.write(data)
    return p


def test_truncated_and_malformed_files(tmp_path):
    raw = open(FIX, "rb").read()
    # truncated data block (TSafeTensorFile.open asserts "Truncated Safetensor file")
    assert "outside the file" in _error(q.safetensors_info, _write(tmp_path, "t.st", raw[:-1]), "blocks.0.norm.scale")
    # header length beyond the file
    bad = (len(raw)).to_bytes(8, "little") + raw[8:]
    assert "header length" in _error(q.safetensors_info, _write(tmp_path, "h.st", bad), "x")
    # too small to hold a header
    assert "too small" in _error(q.safetensors_info, _write(tmp_path, "s.st", b"\0" * 8), "x")
    # malformed JSON
    hj = b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]'  # unterminated
    assert "bad header" in _error(q.safetensors_info, _write(tmp_path, "j.st", len(hj).to_bytes(8, "little") + hj
                                                             + b"\0" * 4), "a")
    # byte size inconsistent with shape
    hj = json.dumps({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}).encode()
    assert "its shape needs" in _error(q.safetensors_info, _write(tmp_path, "z.st", len(hj).to_bytes(8, "little")
                                                                  + hj + b"\0" * 4), "a")


def test_crafted_headers_fail_cleanly(tmp_path):
    """Headers built to overflow the shape or byte products, to pass huge dimensions with an empty
    data range, or to nest without end return a status; nothing wraps, throws or recurses away."""
    import ctypes
    lib = hip.load()

    def st(header):
        hj = json.dumps(header).encode() if isinstance(header, dict) else header
        return _write(tmp_path, "c.st", len(hj).to_bytes(8, "little") + hj + b"\0" * 8)

    # 2^32 * 2^31 elements of F16 wrap a 64-bit byte count to 0, matching an empty data range
    p = st({"w": {"dtype": "F16", "shape": [2 ** 32, 2 ** 31], "data_offsets": [0, 0]}})
    assert "overflows" in _error(q.safetensors_info, p, "w")
    # the element count itself overflows
    p = st({"w": {"dtype": "BF16", "shape": [2 ** 40, 2 ** 30], "data_offsets": [0, 0]}})
    assert "overflows" in _error(q.safetensors_info, p, "w")
    # a zero-sized matrix with a huge row count: consistent bytes, refused before any conversion
    h = ctypes.c_void_p()
    for shape in ([2 ** 30, 0], [0, 8], [8, 2 ** 31]):
        p = st({"w": {"dtype": "F16", "shape": shape, "data_offsets": [0, 2 * shape[0] * shape[1]]}})
        if shape[0] * shape[1] * 2 > 8:
            assert "outside the file" in _error(q.safetensors_info, p, "w")
            continue
        rc = lib.inv_hip_weight_load_safetensors(p.encode(), b"w", None, 0, ctypes.byref(h))
        assert rc == hip.INV_ERR_ARG and "each dimension" in hip.last_error(), shape
    # 200 nested arrays in the metadata: refused, not recursed into
    deep = b'{"__metadata__": ' + b"[" * 200 + b"]" * 200 + b"}"
    assert "bad header" in _error(q.safetensors_info, st(deep), "w")
    shallow = b'{"__metadata__": ' + b"[" * 20 + b"]" * 20 + b', "a": {"dtype": "F32", "shape": [2], ' \
              b'"data_offsets": [0, 8]}}'
    assert q.safetensors_info(st(shallow), "a")["shape"] == (2,)


def test_other_dtypes_are_reported_not_decoded(tmp_path):
    hj = json.dumps({"ids": {"dtype": "I64", "shape": [3], "data_offsets": [0, 24]}}).encode()
    p = _write(tmp_path, "i.st", len(hj).to_bytes(8, "little") + hj + b"\0" * 24)
    info = q.safetensors_info(p, "ids")
    assert info["dtype"] is None and info["shape"] == (3,)


def test_load_rejects_non_matrix_and_bad_bias():
    """Checked before any device work (no GPU needed)."""
    lib = hip.load()
    import ctypes
    h = ctypes.c_void_p()
    rc = lib.inv_hip_weight_load_safetensors(FIX.encode(), b"blocks.0.norm.scale", None, 0, ctypes.byref(h))
    assert rc == hip.INV_ERR_ARG and "2 ([out x in])" in hip.last_error()
    rc = lib.inv_hip_weight_load_safetensors(FIX.encode(), b"blocks.0.attn.qkv.weight", b"blocks.0.norm.scale", 0,
                                             ctypes.byref(h))
    assert rc == hip.INV_ERR_ARG and "24 values" in hip.last_error()
    rc = lib.inv_hip_weight_load_safetensors(FIX.encode(), b"blocks.0.attn.qkv.weight", b"nope", 0, ctypes.byref(h))
    assert rc == hip.INV_ERR_ARG and "no tensor" in hip.last_error()


def test_safetensorfiles_finds_shards_by_index_and_by_search(tmp_path):
    a = os.path.join(tmp_path, "model-00001-of-00002.safetensors")
    b = os.path.join(tmp_path, "model-00002-of-00002.safetensors")
    shutil.copy(FIX, a)
    hj = json.dumps({"extra.weight": {"dtype": "BF16", "shape": [2, 4], "data_offsets": [0, 16]}}).encode()
    _write(tmp_path, os.path.basename(b), len(hj).to_bytes(8, "little") + hj + b"\0" * 16)
    byscan = q.SafeTensorFiles(str(tmp_path))
    assert byscan.find("extra.weight") == b and byscan.find("blocks.0.attn.qkv.weight") == a
    with open(os.path.join(tmp_path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": {"extra.weight": os.path.basename(b),
                                                  "blocks.0.attn.qkv.weight": os.path.basename(a)}}, f)
    byindex = q.SafeTensorFiles(str(tmp_path))
    assert byindex.find("extra.weight") == b and byindex.find("blocks.0.attn.qkv.weight") == a
    with pytest.raises(KeyError):
        byindex.find("not.there")


# ------------------------------------------------------------------ GPU: load --

def _same_products(w_file, w_arr, M=37):
    oracle.rng_seed(5)
    X = oracle.randn_scaled((M, K), 1.0, False)
    y1 = q.linear(as_bf16_bits(X), w_file)
    y2 = q.linear(as_bf16_bits(X), w_arr)
    np.testing.assert_array_equal(y1, y2)
    return y1


@pytest.mark.gpu
def test_bf16_weight_and_f32_bias_from_file(hiplib):
    with q.Weight.from_safetensors(FIX, "blocks.0.attn.qkv.weight", "blocks.0.attn.qkv.bias") as wf, \
            q.Weight(EXP["w_bf16"], EXP["b_f32"]) as wa:
        assert (wf.N, wf.K) == (N, K) and wf.has_bias
        _same_products(wf, wa)


@pytest.mark.gpu
def test_f32_weight_rounded_or_truncated(hiplib):
    w32 = EXP["w32"]
    trunc = oracle.f32_to_bf16_trunc(w32)
    rne = oracle.f32_to_bf16_rne(w32)
    assert np.any(trunc != rne)  # the fixture separates the two roundings
    with q.Weight.from_safetensors(FIX, "blocks.0.mlp.fc32.weight") as wf, q.Weight(rne) as wa:
        y_rne = _same_products(wf, wa)
    with q.Weight.from_safetensors(FIX, "blocks.0.mlp.fc32.weight", truncate=True) as wf, q.Weight(trunc) as wa:
        y_tr = _same_products(wf, wa)
    assert np.any(y_rne != y_tr)


@pytest.mark.gpu
def test_f16_weight_and_bf16_bias(hiplib):
    w = EXP["w16"].astype(np.float32)  # F16 widens exactly, then rounds to bf16
    b = oracle.bf16_to_f32(EXP["b_bf16"])
    with q.Weight.from_safetensors(FIX, "blocks.0.mlp.fc16.weight", "blocks.0.mlp.fc16.bias") as wf, \
            q.Weight(oracle.f32_to_bf16_rne(w), b) as wa:
        _same_products(wf, wa)


# ------------------------------------------------------------ GPU: weight cache --

@pytest.mark.gpu
def test_weight_cache_uploads_once_per_file_and_tensor(hiplib, tmp_path):
    """The reference loads a block's weights from the mapped file on every sampler step and frees
    them (src/quicknn_transformers.pas:1581-1602).  Through the cache, the second and later
    requests of the same tensor (also through the index-JSON shard map) return the resident
    handle: no upload, the same products; free() releases the reference only."""
    q.weight_cache_clear()
    s0 = q.weight_cache_stats()
    a = os.path.join(tmp_path, "model-00001-of-00002.safetensors")
    b = os.path.join(tmp_path, "model-00002-of-00002.safetensors")
    shutil.copy(FIX, a)
    shutil.copy(FIX, b)  # the same bytes in another file: a different cache entry
    with open(os.path.join(tmp_path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": {"blocks.0.attn.qkv.weight": os.path.basename(a),
                                                  "blocks.0.attn.qkv.bias": os.path.basename(a),
                                                  "blocks.0.mlp.fc32.weight": os.path.basename(b)}}, f)
    files = q.SafeTensorFiles(str(tmp_path))
    with q.Weight(EXP["w_bf16"], EXP["b_f32"]) as wa:
        handles = []
        for step in range(3):  # three "sampler steps": load, use, free
            w = files.linear_weight("blocks.0.attn.qkv.weight", "blocks.0.attn.qkv.bias")
            handles.append(w.handle)
            _same_products(w, wa)
            w.free()
        assert len(set(handles)) == 1
    s1 = q.weight_cache_stats()
    wbytes = N * ((K + 7) // 8 * 8) * 2 + N * 4
    assert s1["misses"] - s0["misses"] == 1 and s1["hits"] - s0["hits"] == 2
    assert s1["uploaded_bytes"] - s0["uploaded_bytes"] == wbytes and s1["entries"] == 1
    # another shard, another tensor: one more upload; the bias-less request is its own entry
    w2 = files.linear_weight("blocks.0.mlp.fc32.weight")
    w3 = q.Weight.from_safetensors(a, "blocks.0.attn.qkv.weight", cached=True)
    s2 = q.weight_cache_stats()
    assert s2["misses"] - s1["misses"] == 2 and s2["entries"] == 3
    # a budget evicts unreferenced entries only, least recently used first
    q.weight_cache_set_budget(1)
    assert q.weight_cache_stats()["entries"] == 2  # the qkv weight with bias was released
    w2.free()
    w3.free()
    assert q.weight_cache_stats()["entries"] == 0
    q.weight_cache_set_budget(0)
    # a rewritten file is a new entry (its modification time and size moved)
    w4 = files.linear_weight("blocks.0.attn.qkv.weight", "blocks.0.attn.qkv.bias")
    h4 = w4.handle
    w4.free()
    with open(a, "ab") as f:
        f.write(b"\0" * 8)  # trailing bytes: the header and tensors are unchanged
    w5 = files.linear_weight("blocks.0.attn.qkv.weight", "blocks.0.attn.qkv.bias")
    assert q.weight_cache_stats()["misses"] - s2["misses"] == 2
    w5.free()
    assert h4 is not None
    # clear while referenced: detached, freed on the last release; handles stay usable until then
    w6 = files.linear_weight("blocks.0.mlp.fc32.weight")
    q.weight_cache_clear()
    assert q.weight_cache_stats()["entries"] == 0
    with q.Weight(oracle.f32_to_bf16_rne(EXP["w32"])) as wa:
        _same_products(w6, wa)
    w6.free()
