"""Regenerate the committed fixtures in tests/golden/.

    make -C oracle && python tests/golden/make_golden.py

Fixtures (data only: inputs and expected outputs):
  rng_seed0.json      first outputs of the reference RNG restated
                      (quicknn_sample.pas:212-276) after rng_seed(0) and
                      rng_seed(1234): raw xoshiro256** words and
                      random_normal() values (float32 bit patterns).
  sgemm2_ref.npz      C = A . B^T computed by the reference's own sgemm2.cpp
                      (cpp_sgemm, sgemm2.cpp:530-547) built under oracle/_ref,
                      on bf16-exact inputs drawn from the restated RNG.
                      Requires the reference tree; skipped otherwise.
  linear_small.npz    QNNLinear-shaped cases (bias, SiLU, GELU, ragged
                      shapes) with fp64 closed-form outputs.
  linear_tiny.safetensors + linear_tiny_expected.npz
                      a .safetensors file written byte by byte (u64 LE header
                      length, JSON header, data; the layout TSafeTensorFile.open
                      reads, src/safetensor.pas:466-513) holding BF16, F32 and
                      F16 linear weights and biases plus a __metadata__ entry,
                      and the same arrays with their data byte offsets.
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

SGEMM2_SHAPES = [(4, 8, 128), (12, 20, 256), (33, 17, 384), (8, 40, 300)]
LINEAR_CASES = [
    # (M, K, N, bias, epilogue)
    (16, 64, 48, True, oracle.EPI_NONE),
    (7, 40, 36, True, oracle.EPI_SILU),
    (5, 24, 12, False, oracle.EPI_GELU),
    (33, 19, 21, True, oracle.EPI_NONE),  # K % 8 != 0, N % 4 != 0
    (1, 256, 96, True, oracle.EPI_SILU),
]


def f32_hex(a: np.ndarray) -> list[str]:
    return [f"{int(v):08x}" for v in np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)]


def make_rng() -> dict:
    out = {}
    for seed in (0, 1234):
        oracle.rng_seed(seed)
        state = oracle.rng_state()
        raw = oracle.xoshiro256ss(8)
        oracle.rng_seed(seed)
        normals = oracle.randn(8)
        out[str(seed)] = {"state_after_seed": [f"{s:016x}" for s in state],
                          "xoshiro256ss": [f"{r:016x}" for r in raw],
                          "random_normal_f32": f32_hex(normals)}
    return out


def gen_inputs(seed: int, M: int, K: int, N: int):
    oracle.rng_seed(seed)
    X = oracle.randn_scaled((M, K), 1.0, True)
    W = oracle.randn_scaled((N, K), 0.02, True)
    b = oracle.randn_scaled((N,), 0.01, False)
    return X, W, b


def make_sgemm2(path: str) -> bool:
    if oracle.ref_lib() is None:
        print("oracle/_ref not built (reference tree absent): sgemm2_ref.npz left as is")
        return False
    arrays = {}
    for i, (M, N, K) in enumerate(SGEMM2_SHAPES):
        A, B, _ = gen_inputs(100 + i, M, K, N)
        C = oracle.sgemm2_ref_nt(A, B)
        arrays[f"A{i}"], arrays[f"B{i}"], arrays[f"C{i}"] = A, B, C
    arrays["shapes"] = np.array(SGEMM2_SHAPES, dtype=np.int64)
    np.savez_compressed(path, **arrays)
    return True


def make_linear(path: str) -> None:
    arrays = {}
    for i, (M, K, N, has_bias, epi) in enumerate(LINEAR_CASES):
        X, W, b = gen_inputs(200 + i, M, K, N)
        Wb = oracle.f32_to_bf16_rne(W)
        acc = X.astype(np.float64) @ oracle.bf16_to_f32(Wb).astype(np.float64).T
        if has_bias:
            acc = acc + b.astype(np.float64)
        if epi == oracle.EPI_SILU:
            y = acc / (1.0 + np.exp(-acc))
        elif epi == oracle.EPI_GELU:
            from math import erf, sqrt
            y = 0.5 * acc * (1.0 + np.vectorize(lambda v: erf(v / sqrt(2.0)))(acc))
        else:
            y = acc
        arrays[f"X{i}"], arrays[f"W{i}"], arrays[f"b{i}"], arrays[f"Y{i}"] = X, Wb, b, y
    arrays["cases"] = np.array([(M, K, N, int(hb), epi) for (M, K, N, hb, epi) in LINEAR_CASES], dtype=np.int64)
    np.savez_compressed(path, **arrays)


def make_safetensors(path: str, expected_path: str) -> None:
    """Tensors in file order; F32 weights include exact bf16 ties (low half
    0x8000) and values whose truncation and rounding differ."""
    oracle.rng_seed(77)
    N, K = 12, 24
    w_bf16 = oracle.f32_to_bf16_rne(oracle.randn_scaled((N, K), 0.02, False))
    b_f32 = oracle.randn_scaled((N,), 0.01, False).astype(np.float32)
    w32 = oracle.randn_scaled((N, K), 0.02, False).astype(np.float32)
    bits = w32.view(np.uint32).copy()
    bits[0, :8] = (bits[0, :8] & 0xFFFF0000) | 0x8000          # ties: even and odd upper halves
    bits[1, :8] = (bits[1, :8] & 0xFFFF0000) | 0x7FFF          # just below a tie
    bits[2, :8] = (bits[2, :8] & 0xFFFF0000) | 0x8001          # just above a tie
    w32 = bits.view(np.float32)
    w16 = (oracle.randn_scaled((N, K), 0.02, False)).astype(np.float16)
    b_bf16 = oracle.f32_to_bf16_rne(oracle.randn_scaled((N,), 0.01, False))
    tensors = [
        ("blocks.0.attn.qkv.weight", "BF16", (N, K), w_bf16.astype("<u2").tobytes()),
        ("blocks.0.attn.qkv.bias", "F32", (N,), b_f32.astype("<f4").tobytes()),
        ("blocks.0.mlp.fc32.weight", "F32", (N, K), w32.astype("<f4").tobytes()),
        ("blocks.0.mlp.fc16.weight", "F16", (N, K), w16.astype("<f2").tobytes()),
        ("blocks.0.mlp.fc16.bias", "BF16", (N,), b_bf16.astype("<u2").tobytes()),
        ("blocks.0.norm.scale", "F32", (K,), np.ones(K, "<f4").tobytes()),
    ]
    header, data, offsets = {"__metadata__": {"format": "pt"}}, b"", {}
    for name, dt, shape, raw in tensors:
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [len(data), len(data) + len(raw)]}
        offsets[name] = len(data)
        data += raw
    hj = json.dumps(header, separators=(",", ":")).encode()
    hj += b" " * (-len(hj) % 8)
    with open(path, "wb") as f:
        f.write(len(hj).to_bytes(8, "little") + hj + data)
    base = 8 + len(hj)
    np.savez_compressed(expected_path, w_bf16=w_bf16, b_f32=b_f32, w32=w32, w16=w16, b_bf16=b_bf16,
                        names=np.array([t[0] for t in tensors]),
                        data_offsets=np.array([base + offsets[t[0]] for t in tensors], np.int64))


def main() -> None:
    with open(os.path.join(HERE, "rng_seed0.json"), "w") as f:
        json.dump(make_rng(), f, indent=1)
    make_sgemm2(os.path.join(HERE, "sgemm2_ref.npz"))
    make_linear(os.path.join(HERE, "linear_small.npz"))
    make_safetensors(os.path.join(HERE, "linear_tiny.safetensors"), os.path.join(HERE, "linear_tiny_expected.npz"))
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
