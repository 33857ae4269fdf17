"""Synthetic GGUF inputs for the CLI tests, modelled on the reference's
end-to-end test (tests/test_q4_0.py:28-70) and synthetic model
(tools/dev_make_synth.py:76-112): F32 / F16 / BF16 2-D tensors, a 3-D expert
tensor, passthroughs (1-D norm, a 10x40 tensor whose rows no block divides,
rope_freqs), every KV value type, and a matching imatrix file."""

from __future__ import annotations

import importlib
from pathlib import Path

import numpy as np
import torch

io = importlib.import_module("quant-studio_amd.gguf_io")
GT = importlib.import_module("quant-studio_amd.gguf_types").GGMLQuantizationType
KV, VT = io.KV, io.VT


def bf16_bits(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16) \
        .view(torch.int16).numpy().view(np.uint16)


def small_model(path: Path, seed: int = 42, odd: bool = True) -> dict[str, np.ndarray]:
    """Writes the GGUF; returns the f32 values of every quantizable tensor (numpy order)."""
    rng = np.random.default_rng(seed)
    kvs = [KV("llama.context_length", VT.UINT32, 2048),
           KV("llama.block_count", VT.UINT32, 1),
           KV("llama.attention.head_count", VT.UINT32, 4),
           KV("llama.attention.layer_norm_rms_epsilon", VT.FLOAT32, 1e-5),
           KV("test.flag", VT.BOOL, True),
           KV("test.i8", VT.INT8, -3), KV("test.u16", VT.UINT16, 65000),
           KV("test.i64", VT.INT64, -(1 << 40)), KV("test.f64", VT.FLOAT64, 0.1),
           KV("tokenizer.ggml.tokens", VT.ARRAY, ["<s>", "</s>", "hello"], VT.STRING),
           KV("tokenizer.ggml.scores", VT.ARRAY, [0.0, -1.5, 2.25], VT.FLOAT32),
           KV("general.file_type", VT.UINT32, 32),
           KV("general.name", VT.STRING, "synthetic")]
    tensors, expect = [], {}
    a = rng.standard_normal((200, 256)).astype(np.float32)
    tensors.append(("blk.0.attn_q.weight", (256, 200), GT.F32, a))
    expect["blk.0.attn_q.weight"] = a
    b = (rng.standard_normal((96, 512)) * 0.1).astype(np.float16)
    tensors.append(("blk.0.ffn_up.weight", (512, 96), GT.F16, b))
    expect["blk.0.ffn_up.weight"] = b.astype(np.float32)
    c = rng.standard_normal((80, 256)) * 0.02
    c[0] = 0.0
    c[1] = 0.5
    c[2, 7] = 8.0
    cb = bf16_bits(c)
    tensors.append(("blk.0.attn_k.weight", (256, 80), GT.BF16, cb))
    expect["blk.0.attn_k.weight"] = (cb.astype(np.uint32) << 16).view(np.float32)
    d = (rng.standard_normal((4, 16, 256)) * 0.05).astype(np.float16)
    tensors.append(("blk.0.ffn_gate_exps.weight", (256, 16, 4), GT.F16, d))
    expect["blk.0.ffn_gate_exps.weight"] = d.astype(np.float32)
    tensors.append(("blk.0.attn_norm.weight", (256,), GT.F32,
                    rng.standard_normal(256).astype(np.float32)))
    odd_t = rng.standard_normal((10, 40)).astype(np.float32)
    if odd:
        tensors.append(("blk.0.odd.weight", (40, 10), GT.F32, odd_t))
    tensors.append(("rope_freqs.weight", (32,), GT.F32, rng.standard_normal(32).astype(np.float32)))
    e = bf16_bits(rng.standard_normal((64, 256)) * 0.01)
    tensors.append(("token_embd.weight", (256, 64), GT.BF16, e))
    expect["token_embd.weight"] = (e.astype(np.uint32) << 16).view(np.float32)
    io.write_gguf(path, "llama", kvs, tensors)
    return expect


def imatrix_for(path: Path, names_k: dict[str, int], seed: int = 7, n_mat: dict | None = None,
                zero_frac: float = 0.0, dead_counts: dict | None = None) -> dict:
    """imatrix GGUF: <name>.in_sum2 = v * count per column, <name>.counts = [count].
    zero_frac: that fraction of the columns, and every other 16-column group,
    never fired (in_sum2 = 0); dead_counts: {name: [matrix indices]} whose count
    is 0 (an expert that was never routed: its weights load as 0,
    quant-studio.py:80-85)."""
    rng = np.random.default_rng(seed)
    tensors, values = [], {}
    for name, k in names_k.items():
        m = (n_mat or {}).get(name, 1)
        v = (rng.random(k * m).astype(np.float32) * 4.0 + 0.05)
        if zero_frac:
            v[rng.random(k * m) < zero_frac] = 0.0
            v.reshape(-1, 16)[::2] = 0.0
        cnt = np.full(m, 100.0, np.float32)
        cnt[list((dead_counts or {}).get(name, []))] = 0.0
        s = (v.reshape(m, k) * cnt[:, None]).astype(np.float32).reshape(-1)
        tensors.append((name + ".in_sum2", (k * m,), GT.F32, s))
        tensors.append((name + ".counts", (m,), GT.F32, cnt))
        live = cnt[:, None] > 0
        values[name] = np.where(live, s.reshape(m, k) / np.where(live, cnt[:, None], 1), 0).reshape(-1)
    io.write_gguf(path, "imatrix", [KV("general.type", VT.STRING, "imatrix")], tensors)
    return values


def fallback_model(path: Path) -> dict[str, np.ndarray]:
    """Tensors whose rows (288 values) are a multiple of 32 but not of 256."""
    rng = np.random.default_rng(3)
    names = ["blk.0.attn_q.weight", "blk.0.attn_k.weight", "blk.0.attn_v.weight",
             "blk.0.ffn_down.weight", "blk.0.ffn_up.weight"]
    arrays = {n: (rng.standard_normal((48, 288)) * 0.02).astype(np.float32) for n in names}
    io.write_gguf(path, "llama", [KV("llama.block_count", VT.UINT32, 1)],
                  [(n, (288, 48), GT.F32, a) for n, a in arrays.items()])
    return arrays
