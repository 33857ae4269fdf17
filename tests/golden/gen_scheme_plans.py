#!/usr/bin/env python3
"""Write golden per-tensor type plans from the reference's policy module.

Runs ONLY in the build container, where the reference checkout is mounted at
/root/reference. Imports kernels/scheme.py (the llama-quantize mix policy the
reference follows) with a stand-in `gguf` module that supplies only enum
names and the public GGML block sizes, and records the plan that
scheme.decide_types() / tensor_requires_imatrix() produce for a matrix of
synthetic models x every scheme x imatrix / --pure / type-override options.
Nothing from the reference is stored except those decisions
(scheme_plans.json.gz next to this script; a trailing '*' on a
type marks tensor_requires_imatrix).

Usage: python tests/golden/gen_scheme_plans.py [--ref /root/reference]
"""

from __future__ import annotations

import argparse
import enum
import gzip
import json
import sys
import types
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
from gen_golden import FILE_TYPES, GGML_TYPES  # noqa: E402

# Q1_0 / Q2_0 exist only by name in the policy's option table; give them ids
# outside the public range so the stand-in enums are complete.
EXTRA_TYPES = dict(Q1_0=100, Q2_0=101)
EXTRA_FILE_TYPES = dict(MOSTLY_Q1_0=100, MOSTLY_Q2_0=101)
# (block size, type size) from the public GGML type table
QUANT_SIZES = dict(F32=(1, 4), F16=(1, 2), Q4_0=(32, 18), Q4_1=(32, 20), Q5_0=(32, 22),
                   Q5_1=(32, 24), Q8_0=(32, 34), Q8_1=(32, 36), Q2_K=(256, 84), Q3_K=(256, 110),
                   Q4_K=(256, 144), Q5_K=(256, 176), Q6_K=(256, 210), Q8_K=(256, 292),
                   IQ2_XXS=(256, 66), IQ2_XS=(256, 74), IQ3_XXS=(256, 98), IQ1_S=(256, 50),
                   IQ4_NL=(32, 18), IQ3_S=(256, 110), IQ2_S=(256, 82), IQ4_XS=(256, 136),
                   I8=(1, 1), I16=(1, 2), I32=(1, 4), I64=(1, 8), F64=(1, 8), IQ1_M=(256, 56),
                   BF16=(1, 2), TQ1_0=(256, 54), TQ2_0=(256, 66), MXFP4=(32, 17),
                   Q1_0=(128, 18), Q2_0=(64, 18))


def install_enum_module() -> None:
    g = types.ModuleType("gguf")
    c = types.ModuleType("gguf.constants")
    GT = enum.IntEnum("GGMLQuantizationType", {**GGML_TYPES, **EXTRA_TYPES})
    FT = enum.IntEnum("LlamaFileType", {**FILE_TYPES, **EXTRA_FILE_TYPES})
    g.GGMLQuantizationType = GT
    c.LlamaFileType = FT
    g.LlamaFileType = FT
    c.GGML_QUANT_SIZES = {GT[k]: v for k, v in QUANT_SIZES.items()}
    g.GGML_QUANT_SIZES = c.GGML_QUANT_SIZES
    g.GGML_QUANT_VERSION = 2
    g.constants = c
    sys.modules["gguf"] = g
    sys.modules["gguf.constants"] = c


def dense_layers(n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim, qkv=False, q_norm=False):
    t = []
    for i in range(n_layer):
        p = f"blk.{i}."
        t.append((p + "attn_norm.weight", (n_embd,)))
        if qkv:
            t.append((p + "attn_qkv.weight", (n_embd, (n_head + 2 * n_head_kv) * head_dim)))
        else:
            t.append((p + "attn_q.weight", (n_embd, n_head * head_dim)))
            t.append((p + "attn_k.weight", (n_embd, n_head_kv * head_dim)))
            t.append((p + "attn_v.weight", (n_embd, n_head_kv * head_dim)))
        if q_norm:
            t.append((p + "attn_q_norm.weight", (head_dim,)))
            t.append((p + "attn_k_norm.weight", (head_dim,)))
        t.append((p + "attn_output.weight", (n_head * head_dim, n_embd)))
        t.append((p + "ffn_norm.weight", (n_embd,)))
        t.append((p + "ffn_gate.weight", (n_embd, n_ff)))
        t.append((p + "ffn_up.weight", (n_embd, n_ff)))
        t.append((p + "ffn_down.weight", (n_ff, n_embd)))
    return t


def models():
    """(name, ModelInfo fields, [(tensor name, ggml shape ne)]) in file order."""
    ms = []
    # 36-layer Qwen3-like model with tied embeddings (the 4B-class benchmark model)
    t = [("token_embd.weight", (2560, 151936))] + dense_layers(36, 2560, 9728, 32, 8, 128, q_norm=True)
    t.append(("output_norm.weight", (2560,)))
    ms.append(("qwen3_36l_tied", dict(arch="qwen3", n_layer=36, n_expert=0, n_head=32, n_head_kv=8,
                                      is_70b=False), t))
    # small llama, untied output, n_gqa = 1 (the reference's synthetic test model shape)
    t = [("token_embd.weight", (256, 512))] + dense_layers(2, 256, 512, 8, 8, 32)
    t += [("output_norm.weight", (256,)), ("output.weight", (256, 512))]
    ms.append(("llama_2l", dict(arch="llama", n_layer=2, n_expert=0, n_head=8, n_head_kv=8,
                                is_70b=False), t))
    # 80-layer llama (the 70B special cases), small widths to keep the list cheap
    t = [("token_embd.weight", (512, 1024))] + dense_layers(80, 512, 1024, 64, 8, 8)
    t += [("output_norm.weight", (512,)), ("output.weight", (512, 1024))]
    ms.append(("llama_80l", dict(arch="llama", n_layer=80, n_expert=0, n_head=64, n_head_kv=8,
                                 is_70b=True), t))
    # falcon with fused qkv
    t = [("token_embd.weight", (512, 2048))] + dense_layers(8, 512, 2048, 8, 1, 64, qkv=True)
    t += [("output_norm.weight", (512,)), ("output.weight", (512, 2048))]
    ms.append(("falcon_8l", dict(arch="falcon", n_layer=8, n_expert=0, n_head=8, n_head_kv=1,
                                 is_70b=False), t))
    # 8-expert MoE with kv_b and expert tensors (3-D), layer from the tensor name
    t = [("token_embd.weight", (512, 1024))]
    for i in range(6):
        p = f"blk.{i}."
        t += [(p + "attn_norm.weight", (512,)), (p + "attn_q.weight", (512, 512)),
              (p + "attn_kv_b.weight", (256, 1024)), (p + "attn_k.weight", (512, 128)),
              (p + "attn_output.weight", (512, 512)), (p + "ffn_gate_inp.weight", (512, 8)),
              (p + "ffn_gate_exps.weight", (512, 256, 8)), (p + "ffn_up_exps.weight", (512, 256, 8)),
              (p + "ffn_down_exps.weight", (256, 512, 8))]
    t += [("output_norm.weight", (512,)), ("output.weight", (512, 1024))]
    ms.append(("moe_8x", dict(arch="deepseek2", n_layer=6, n_expert=8, n_head=16, n_head_kv=16,
                              is_70b=False), t))
    # shape fallbacks and never-quantized names
    t = [("token_embd.weight", (288, 100)), ("blk.0.attn_q.weight", (288, 288)),
         ("blk.0.attn_v.weight", (40, 64)), ("blk.0.ffn_down.weight", (2592, 256)),
         ("blk.0.ffn_up.weight", (256, 2592)), ("blk.0.time_mix_first.weight", (256, 256)),
         ("position_embd.weight", (256, 64)), ("blk.0.attn_norm.weight", (288,)),
         ("blk.0.ssm_conv1d.weight", (4, 256)), ("blk.0.some.bias", (256, 4)),
         ("blk.0.ffn_gate.weight", (256, 2592))]
    ms.append(("odd_shapes", dict(arch="llama", n_layer=1, n_expert=0, n_head=4, n_head_kv=4,
                                  is_70b=False), t))
    return ms


OPTIONS = [
    dict(),
    dict(imatrix=True),
    dict(pure=True),
    dict(imatrix=True, tet="Q4_0"),
    dict(imatrix=True, ott="Q8_0", tet="Q6_K"),
    dict(imatrix=True, tt=[["attn_v", "Q8_0"], ["ffn_down\\.weight", "Q5_K"]]),
    dict(leave_output=True),
]


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    args = ap.parse_args()
    install_enum_module()
    sys.path.insert(0, args.ref)
    import importlib
    scheme = importlib.import_module("kernels.scheme")
    GT = sys.modules["gguf"].GGMLQuantizationType

    records = []
    for mname, info, tensors in models():
        model = scheme.ModelInfo(**info)
        names = [n for n, _ in tensors]
        for opt in scheme.QUANT_OPTIONS:
            for o in OPTIONS:
                tt = [(p, GT[t]) for p, t in o.get("tt", [])]
                tet = GT[o["tet"]] if "tet" in o else None
                ott = GT[o["ott"]] if "ott" in o else None
                rec = dict(model=mname, scheme=opt.name, options=o)
                try:
                    qs = scheme.init_state(model, names, bool(o.get("imatrix")), tt)
                    plan = []
                    for name, ne in tensors:
                        dst = scheme.tensor_get_type(
                            qs, model, name, ne, GT.BF16, opt.ftype, pure=bool(o.get("pure")),
                            quantize_output_tensor=not o.get("leave_output"),
                            token_embedding_type=tet, output_tensor_type=ott)
                        req = scheme.tensor_requires_imatrix(name, dst, opt.ftype)
                        plan.append(f"{dst.name}{'*' if req else ''}")
                    rec["plan"] = " ".join(plan)
                    rec["n_fallback"] = qs.n_fallback
                except Exception as e:  # the policy's own errors are part of the record
                    rec["error"] = f"{type(e).__name__}: {e}"
                records.append(rec)
    out = dict(models=[dict(name=m, info=i, tensors=[[n, list(ne)] for n, ne in t])
                       for m, i, t in models()],
               options_table=[dict(name=o.name, ftype=o.ftype.name,
                                   default=(o.default_type.name if o.default_type is not None else None))
                              for o in scheme.QUANT_OPTIONS],
               records=records)
    with gzip.open(HERE / "scheme_plans.json.gz", "wt") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"{len(records)} plans written")


if __name__ == "__main__":
    main()
