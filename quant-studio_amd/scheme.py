"""Tensor-type policy: which ggml type each tensor of a model gets for a scheme.

Restates the reference's llama-quantize mix policy (kernels/scheme.py:1-644,
itself a mirror of llama.cpp's llama-quant.cpp at a pinned commit):
QUANT_OPTIONS (scheme.py:55-95), the default type per file type (:123-160),
tensor categories (:168-226), never-quantized names (:234-268), the
per-layer counters (:313-340), the mixture rules (:387-563), the shape
fallbacks (:364-384) and the imatrix requirement (:605-614).

The decisions are stateful and order-dependent: build a QuantState over all
tensor names, then call tensor_get_type() per tensor in loader order
(weight_name_key). Parity: tests/test_scheme.py replays plans recorded from the
reference (tests/golden/scheme_plans.json.gz).
"""

from __future__ import annotations

import re
import sys
from dataclasses import dataclass, field
from enum import Enum

from .gguf_types import GGMLQuantizationType as GT
from .gguf_types import LlamaFileType as FT
from .gguf_types import QUANT_SIZES

POLICY_COMMIT = "9871d51fd7a6a4fb300100ed236f3962e72fd6ee"   # llama.cpp, as pinned by the reference


# ---------------------------------------------------------------------------
# schemes
# ---------------------------------------------------------------------------

# file type -> default tensor type (llama_ftype_get_default_type)
DEFAULT_TYPE: dict[FT, GT] = {
    FT.MOSTLY_Q4_0: GT.Q4_0, FT.MOSTLY_Q4_1: GT.Q4_1, FT.MOSTLY_Q5_0: GT.Q5_0,
    FT.MOSTLY_Q5_1: GT.Q5_1, FT.MOSTLY_Q8_0: GT.Q8_0, FT.MOSTLY_F16: GT.F16,
    FT.MOSTLY_BF16: GT.BF16, FT.ALL_F32: GT.F32, FT.MOSTLY_Q1_0: GT.Q1_0,
    FT.MOSTLY_Q2_0: GT.Q2_0, FT.MOSTLY_MXFP4_MOE: GT.MXFP4,
    FT.MOSTLY_Q2_K_S: GT.Q2_K, FT.MOSTLY_Q2_K: GT.Q2_K, FT.MOSTLY_IQ3_XS: GT.IQ3_S,
    FT.MOSTLY_Q3_K_S: GT.Q3_K, FT.MOSTLY_Q3_K_M: GT.Q3_K, FT.MOSTLY_Q3_K_L: GT.Q3_K,
    FT.MOSTLY_Q4_K_S: GT.Q4_K, FT.MOSTLY_Q4_K_M: GT.Q4_K,
    FT.MOSTLY_Q5_K_S: GT.Q5_K, FT.MOSTLY_Q5_K_M: GT.Q5_K, FT.MOSTLY_Q6_K: GT.Q6_K,
    FT.MOSTLY_TQ1_0: GT.TQ1_0, FT.MOSTLY_TQ2_0: GT.TQ2_0,
    FT.MOSTLY_IQ2_XXS: GT.IQ2_XXS, FT.MOSTLY_IQ2_XS: GT.IQ2_XS,
    FT.MOSTLY_IQ2_S: GT.IQ2_XS,        # the IQ2_S scheme's default tensors are IQ2_XS
    FT.MOSTLY_IQ2_M: GT.IQ2_S, FT.MOSTLY_IQ3_XXS: GT.IQ3_XXS,
    FT.MOSTLY_IQ1_S: GT.IQ1_S, FT.MOSTLY_IQ1_M: GT.IQ1_M, FT.MOSTLY_IQ4_NL: GT.IQ4_NL,
    FT.MOSTLY_IQ4_XS: GT.IQ4_XS, FT.MOSTLY_IQ3_S: GT.IQ3_S, FT.MOSTLY_IQ3_M: GT.IQ3_S,
}


@dataclass(frozen=True)
class QuantOption:
    name: str
    ftype: FT
    desc: str

    @property
    def default_type(self) -> GT | None:
        return DEFAULT_TYPE.get(self.ftype)

    @property
    def supported(self) -> bool:
        """A HIP quantizer exists for the scheme's default tensor type."""
        if self.name == "COPY" or self.default_type is None:
            return False
        return self.default_type in _kernel_types()


# name, file type, description: llama-quantize's option table (the CLI contract)
QUANT_OPTIONS: list[QuantOption] = [QuantOption(n, FT[f], d) for n, f, d in (
    ("Q1_0", "MOSTLY_Q1_0", "1.125 bpw quantization"),
    ("Q2_0", "MOSTLY_Q2_0", "2.25 bpw quantization (group 64)"),
    ("Q4_0", "MOSTLY_Q4_0", "4.34G, +0.4685 ppl @ Llama-3-8B"),
    ("Q4_1", "MOSTLY_Q4_1", "4.78G, +0.4511 ppl @ Llama-3-8B"),
    ("MXFP4_MOE", "MOSTLY_MXFP4_MOE", "MXFP4 MoE"),
    ("Q5_0", "MOSTLY_Q5_0", "5.21G, +0.1316 ppl @ Llama-3-8B"),
    ("Q5_1", "MOSTLY_Q5_1", "5.65G, +0.1062 ppl @ Llama-3-8B"),
    ("IQ2_XXS", "MOSTLY_IQ2_XXS", "2.06 bpw quantization"),
    ("IQ2_XS", "MOSTLY_IQ2_XS", "2.31 bpw quantization"),
    ("IQ2_S", "MOSTLY_IQ2_S", "2.5  bpw quantization"),
    ("IQ2_M", "MOSTLY_IQ2_M", "2.7  bpw quantization"),
    ("IQ1_S", "MOSTLY_IQ1_S", "1.56 bpw quantization"),
    ("IQ1_M", "MOSTLY_IQ1_M", "1.75 bpw quantization"),
    ("TQ1_0", "MOSTLY_TQ1_0", "1.69 bpw ternarization"),
    ("TQ2_0", "MOSTLY_TQ2_0", "2.06 bpw ternarization"),
    ("Q2_K", "MOSTLY_Q2_K", "2.96G, +3.5199 ppl @ Llama-3-8B"),
    ("Q2_K_S", "MOSTLY_Q2_K_S", "2.96G, +3.1836 ppl @ Llama-3-8B"),
    ("IQ3_XXS", "MOSTLY_IQ3_XXS", "3.06 bpw quantization"),
    ("IQ3_S", "MOSTLY_IQ3_S", "3.44 bpw quantization"),
    ("IQ3_M", "MOSTLY_IQ3_M", "3.66 bpw quantization mix"),
    ("Q3_K", "MOSTLY_Q3_K_M", "alias for Q3_K_M"),
    ("IQ3_XS", "MOSTLY_IQ3_XS", "3.3 bpw quantization"),
    ("Q3_K_S", "MOSTLY_Q3_K_S", "3.41G, +1.6321 ppl @ Llama-3-8B"),
    ("Q3_K_M", "MOSTLY_Q3_K_M", "3.74G, +0.6569 ppl @ Llama-3-8B"),
    ("Q3_K_L", "MOSTLY_Q3_K_L", "4.03G, +0.5562 ppl @ Llama-3-8B"),
    ("IQ4_NL", "MOSTLY_IQ4_NL", "4.50 bpw non-linear quantization"),
    ("IQ4_XS", "MOSTLY_IQ4_XS", "4.25 bpw non-linear quantization"),
    ("Q4_K", "MOSTLY_Q4_K_M", "alias for Q4_K_M"),
    ("Q4_K_S", "MOSTLY_Q4_K_S", "4.37G, +0.2689 ppl @ Llama-3-8B"),
    ("Q4_K_M", "MOSTLY_Q4_K_M", "4.58G, +0.1754 ppl @ Llama-3-8B"),
    ("Q5_K", "MOSTLY_Q5_K_M", "alias for Q5_K_M"),
    ("Q5_K_S", "MOSTLY_Q5_K_S", "5.21G, +0.1049 ppl @ Llama-3-8B"),
    ("Q5_K_M", "MOSTLY_Q5_K_M", "5.33G, +0.0569 ppl @ Llama-3-8B"),
    ("Q6_K", "MOSTLY_Q6_K", "6.14G, +0.0217 ppl @ Llama-3-8B"),
    ("Q8_0", "MOSTLY_Q8_0", "7.96G, +0.0026 ppl @ Llama-3-8B"),
    ("F16", "MOSTLY_F16", "14.00G, +0.0020 ppl @ Mistral-7B"),
    ("BF16", "MOSTLY_BF16", "14.00G, -0.0050 ppl @ Mistral-7B"),
    ("F32", "ALL_F32", "26.00G              @ 7B"),
    ("COPY", "ALL_F32", "only copy tensors, no quantizing"),
)]


def _kernel_types() -> set[GT]:
    from . import QUANT_TYPES
    return {s.ggml_type for s in QUANT_TYPES.values()}


def parse_scheme(name: str) -> QuantOption | None:
    up = name.upper()
    return next((o for o in QUANT_OPTIONS if o.name == up), None)


def format_scheme_table() -> str:
    rows = [f"quantization schemes (llama.cpp {POLICY_COMMIT[:10]}), [x] = a HIP quantizer exists"]
    for o in QUANT_OPTIONS:
        dt = o.default_type
        rows.append(f"  [{'x' if o.supported else ' '}] {o.name:10s} default "
                    f"{dt.name if dt is not None else '-':8s} {o.desc}")
    return "\n".join(rows)


# ---------------------------------------------------------------------------
# tensors
# ---------------------------------------------------------------------------

class Cat(Enum):
    OUTPUT = 0
    TOKEN_EMBD = 1
    ATTN_QKV = 2
    ATTN_KV_B = 3
    ATTN_V = 4
    ATTN_K = 5
    ATTN_Q = 6
    ATTN_OUTPUT = 7
    FFN_UP = 8
    FFN_GATE = 9
    FFN_DOWN = 10
    OTHER = 11


_TOKEN_EMBD_NAMES = ("token_embd.weight", "per_layer_token_embd.weight")
# substring -> category, first match wins (after the exact output/token names)
_CAT_BY_SUBSTRING = (("attn_qkv.weight", Cat.ATTN_QKV), ("attn_kv_b.weight", Cat.ATTN_KV_B),
                     ("attn_v.weight", Cat.ATTN_V), ("attn_k.weight", Cat.ATTN_K),
                     ("attn_q.weight", Cat.ATTN_Q), ("attn_output.weight", Cat.ATTN_OUTPUT),
                     ("ffn_up", Cat.FFN_UP), ("ffn_gate", Cat.FFN_GATE), ("ffn_down", Cat.FFN_DOWN))


def category(name: str) -> Cat:
    if name == "output.weight":
        return Cat.OUTPUT
    if name in _TOKEN_EMBD_NAMES:
        return Cat.TOKEN_EMBD
    for sub, cat in _CAT_BY_SUBSTRING:
        if sub in name:
            return cat
    return Cat.OTHER


def is_attn_v_like(cat: Cat) -> bool:
    return cat in (Cat.ATTN_V, Cat.ATTN_QKV, Cat.ATTN_KV_B)


def weight_name_key(name: str) -> tuple[int, str]:
    """Loader order: block number (non-block tensors first), then name."""
    m = re.match(r"blk\.(\d+)\.", name)
    return (int(m.group(1)) if m else -1, name)


# name fragments of tensors that are never quantized
_NEVER_QUANTIZE = (
    "_norm.weight", "ffn_gate_inp.weight", "ffn_gate_tid2eid.weight",
    "altup", "laurel", "per_layer_model_proj", "ssm_conv1d", "shortconv.conv.weight",
    "indexer.k_proj.weight", "indexer.q_proj.weight",
    "time_mix_first.weight", "time_mix_w0.weight", "time_mix_w1.weight", "time_mix_w2.weight",
    "time_mix_v0.weight", "time_mix_v1.weight", "time_mix_v2.weight",
    "time_mix_a0.weight", "time_mix_a1.weight", "time_mix_a2.weight",
    "time_mix_g1.weight", "time_mix_g2.weight", "time_mix_decay_w1.weight",
    "time_mix_decay_w2.weight", "time_mix_lerp_fused.weight", "attn_rel_b.weight",
    ".position_embd", "sam.pos_embd", "sam.neck.", "sam.net_", ".rel_pos", ".patch_embd",
    ".patch_merger", "a.rvq.codebook", "mm.a.code_embd",
)


def allows_quantization(name: str, n_dims: int, quantize_output: bool = True,
                        only_copy: bool = False) -> bool:
    if only_copy or n_dims < 2 or not name.endswith("weight"):
        return False
    if name == "output.weight" and not quantize_output:
        return False
    if name in ("position_embd.weight", "token_types.weight"):
        return False
    return not any(s in name for s in _NEVER_QUANTIZE)


_UNQUANTIZED = {GT.F32, GT.F16, GT.BF16, GT.F64, GT.I8, GT.I16, GT.I32, GT.I64}


def is_quantized(t: GT) -> bool:
    return t not in _UNQUANTIZED


def block_size(t: GT) -> int:
    return QUANT_SIZES[t][0]


# ---------------------------------------------------------------------------
# model facts and counters
# ---------------------------------------------------------------------------

@dataclass
class ModelInfo:
    arch: str = ""
    n_layer: int = 0
    n_expert: int = 0
    n_head: int = 0
    n_head_kv: int = 0
    is_70b: bool = False        # llama with 80 layers

    @property
    def n_gqa(self) -> int:
        return self.n_head // self.n_head_kv if self.n_head_kv > 0 else 0

    @classmethod
    def from_kv(cls, kv: dict) -> "ModelInfo":
        """From a GGUF key/value dict (first layer's value for per-layer arrays)."""
        arch = kv["general.architecture"]

        def get(suffix, default=0):
            v = kv.get(f"{arch}.{suffix}", default)
            return int(v[0]) if isinstance(v, list) else int(v)

        n_layer, n_head = get("block_count"), get("attention.head_count")
        return cls(arch=arch, n_layer=n_layer, n_expert=get("expert_count"), n_head=n_head,
                   n_head_kv=get("attention.head_count_kv", n_head),
                   is_70b=(arch == "llama" and n_layer == 80))


@dataclass
class QuantState:
    n_attention_wv: int = 0
    n_ffn_down: int = 0
    n_ffn_gate: int = 0
    n_ffn_up: int = 0
    i_attention_wv: int = 0
    i_ffn_down: int = 0
    i_ffn_gate: int = 0
    i_ffn_up: int = 0
    n_fallback: int = 0
    has_imatrix: bool = False
    has_tied_embeddings: bool = True
    overrides: list = field(default_factory=list)     # [(compiled regex, GT)]


def init_state(model: ModelInfo, names: list[str], has_imatrix: bool,
               overrides: list[tuple[str, GT]] | None = None) -> QuantState:
    st = QuantState(has_imatrix=has_imatrix)
    st.n_attention_wv = sum(1 for n in names if is_attn_v_like(category(n)))
    st.has_tied_embeddings = "output.weight" not in names
    st.n_ffn_down = st.n_ffn_gate = st.n_ffn_up = model.n_layer
    st.overrides = [(re.compile(p), t) for p, t in (overrides or [])]
    return st


def use_more_bits(i: int, n: int) -> bool:
    return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2


def _layer(counter: int, n: int, name: str, model: ModelInfo) -> tuple[int, int]:
    """Layer index of a per-layer tensor: the running counter, or for MoE models
    (whose expert tensors are not consecutive) the number in the name."""
    if max(1, model.n_expert) > 1:
        m = re.match(r"blk\.(\d+)\.", name)
        if m is None:
            raise ValueError(f"failed to determine layer for tensor {name}")
        counter = int(m.group(1))
        if not 0 <= counter < n:
            raise ValueError(f"bad layer {counter} for tensor {name}")
    return counter, n


_FALLBACK = {
    GT.IQ1_S: GT.IQ4_NL, GT.IQ1_M: GT.IQ4_NL, GT.IQ2_XXS: GT.IQ4_NL, GT.IQ2_XS: GT.IQ4_NL,
    GT.IQ2_S: GT.IQ4_NL, GT.IQ3_XXS: GT.IQ4_NL, GT.IQ3_S: GT.IQ4_NL, GT.IQ4_XS: GT.IQ4_NL,
    GT.Q2_0: GT.Q4_0, GT.Q2_K: GT.Q4_0, GT.Q3_K: GT.Q4_0, GT.TQ1_0: GT.Q4_0, GT.TQ2_0: GT.Q4_0,
    GT.Q4_K: GT.Q5_0, GT.Q5_K: GT.Q5_1, GT.Q6_K: GT.Q8_0,
}


def shape_fallback(st: QuantState, name: str, ncols: int, target: GT) -> GT:
    """A row length the target's block does not divide falls back to a
    smaller-block type (F16 when even that does not fit)."""
    if ncols % block_size(target) == 0:
        return target
    st.n_fallback += 1
    if target not in _FALLBACK:
        raise ValueError(f"no tensor type fallback is defined for type {target.name}")
    ret = _FALLBACK[target]
    if ncols % block_size(ret):
        ret = GT.F16
    print(f"warning: {name}: ncols {ncols} not divisible by {block_size(target)} "
          f"(required for {target.name}) -> falling back to {ret.name}", file=sys.stderr)
    return ret


# ---------------------------------------------------------------------------
# the mixture rules, one function per tensor family
# ---------------------------------------------------------------------------

_IQ2_LIKE = (FT.MOSTLY_IQ2_XXS, FT.MOSTLY_IQ2_XS, FT.MOSTLY_IQ1_S, FT.MOSTLY_IQ2_S,
             FT.MOSTLY_IQ2_M, FT.MOSTLY_IQ1_M)
_IQ2_S_M = (FT.MOSTLY_IQ2_S, FT.MOSTLY_IQ2_M)


def _rule_output(t: GT, ftype: FT, model: ModelInfo, ncols: int, out_type: GT | None) -> GT:
    if out_type is not None:
        return out_type
    if ftype == FT.MOSTLY_MXFP4_MOE or model.arch == "falcon" or ncols % block_size(t):
        return GT.Q8_0
    if ftype in (FT.MOSTLY_IQ2_XXS, FT.MOSTLY_IQ2_XS, FT.MOSTLY_IQ3_XXS, FT.MOSTLY_IQ1_S,
                 FT.MOSTLY_IQ2_S, FT.MOSTLY_IQ2_M, FT.MOSTLY_IQ1_M):
        return GT.Q5_K
    return t if t == GT.Q8_0 else GT.Q6_K


def _rule_token_embd(t: GT, ftype: FT, emb_type: GT | None) -> GT:
    if emb_type is not None:
        return emb_type
    if ftype in (FT.MOSTLY_IQ2_XXS, FT.MOSTLY_IQ2_XS, FT.MOSTLY_IQ1_S, FT.MOSTLY_IQ1_M):
        return GT.Q2_K
    if ftype in _IQ2_S_M or ftype == FT.MOSTLY_IQ3_XXS:
        return GT.IQ3_S
    if ftype in (FT.MOSTLY_TQ1_0, FT.MOSTLY_TQ2_0, FT.MOSTLY_Q2_0):
        return GT.Q4_K
    return t


def _rule_iq2_family(st: QuantState, t: GT, ftype: FT, model: ModelInfo, cat: Cat) -> GT:
    """Schemes at ~2 bpw (IQ1/IQ2): protect attn_v, the first ffn_down layers, attn_output."""
    if is_attn_v_like(cat):
        if model.n_gqa >= 4 or model.n_expert >= 4:
            t = GT.Q4_K
        else:
            t = GT.IQ3_S if ftype in _IQ2_S_M else GT.Q2_K
        st.i_attention_wv += 1
    elif model.n_expert == 8 and cat == Cat.ATTN_K:
        t = GT.Q4_K
    elif cat == Cat.FFN_DOWN:
        if st.i_ffn_down < st.n_ffn_down // 8:
            t = GT.IQ3_S if ftype in _IQ2_S_M else GT.Q2_K
        st.i_ffn_down += 1
    elif cat == Cat.ATTN_OUTPUT:
        if model.n_expert == 8:
            t = GT.Q5_K
        elif ftype in (FT.MOSTLY_IQ1_S, FT.MOSTLY_IQ1_M):
            t = GT.IQ2_XXS
        elif ftype in _IQ2_S_M:
            t = GT.IQ3_S
    return t


def _rule_attn_v(st: QuantState, t: GT, ftype: FT, model: ModelInfo) -> GT:
    gqa4 = model.n_gqa >= 4
    if ftype == FT.MOSTLY_Q2_K:
        t = GT.Q4_K if gqa4 else GT.Q3_K
    elif ftype == FT.MOSTLY_Q2_K_S and gqa4:
        t = GT.Q4_K
    elif ftype == FT.MOSTLY_IQ3_XXS:
        t = GT.Q4_K if gqa4 else (GT.IQ3_XXS if st.has_imatrix else GT.IQ3_S)
    elif ftype in (FT.MOSTLY_IQ3_XS, FT.MOSTLY_IQ3_S) and gqa4:
        t = GT.Q4_K
    elif ftype == FT.MOSTLY_IQ3_M:
        t = GT.Q4_K
    elif ftype == FT.MOSTLY_Q3_K_M:
        t = GT.Q5_K if st.i_attention_wv < 2 else GT.Q4_K
    elif ftype == FT.MOSTLY_Q3_K_L:
        t = GT.Q5_K
    elif ftype in (FT.MOSTLY_IQ4_NL, FT.MOSTLY_IQ4_XS) and gqa4:
        t = GT.Q5_K
    elif ftype in (FT.MOSTLY_Q4_K_M, FT.MOSTLY_Q5_K_M) and \
            use_more_bits(st.i_attention_wv, st.n_attention_wv):
        t = GT.Q6_K
    elif ftype == FT.MOSTLY_Q4_K_S and st.i_attention_wv < 4:
        t = GT.Q5_K
    if model.is_70b and t in (GT.Q3_K, GT.Q4_K):
        t = GT.Q5_K            # attn_v is 8x smaller than attn_q there: extra bits are cheap
    if model.n_expert == 8:
        t = GT.Q8_0
    st.i_attention_wv += 1
    return t


def _rule_ffn_down(st: QuantState, t: GT, ftype: FT, model: ModelInfo, name: str) -> GT:
    i, n = _layer(st.i_ffn_down, st.n_ffn_down, name, model)
    falcon = model.arch == "falcon"
    if ftype == FT.MOSTLY_Q2_K:
        t = GT.Q3_K
    elif ftype == FT.MOSTLY_Q2_K_S:
        if i < n // 8:
            t = GT.Q4_K
    elif ftype == FT.MOSTLY_IQ3_XXS and not st.has_imatrix:
        t = GT.Q4_K if i < n // 8 else GT.Q3_K
    elif ftype == FT.MOSTLY_Q3_K_M:
        if i < n // 16:
            t = GT.Q5_K
        elif not falcon or use_more_bits(i, n):
            t = GT.Q4_K
        else:
            t = GT.Q3_K
    elif ftype == FT.MOSTLY_IQ3_M and (i < n // 8 or (model.n_expert == 8 and use_more_bits(i, n))):
        t = GT.Q4_K
    elif ftype == FT.MOSTLY_Q3_K_L:
        t = GT.Q4_K if falcon else GT.Q5_K
    elif ftype == FT.MOSTLY_Q4_K_M:
        if falcon:
            t = GT.Q6_K if i < n // 16 else (GT.Q5_K if use_more_bits(i, n) else GT.Q4_K)
        elif use_more_bits(i, n):
            t = GT.Q6_K
    elif i < n // 8 and ftype in (FT.MOSTLY_IQ4_NL, FT.MOSTLY_IQ4_XS) and not st.has_imatrix:
        t = GT.Q5_K
    elif ftype == FT.MOSTLY_Q5_K_M and use_more_bits(i, n):
        t = GT.Q6_K
    elif ftype == FT.MOSTLY_Q4_K_S and not falcon and i < n // 8:
        t = GT.Q5_K
    elif ftype in (FT.MOSTLY_Q4_0, FT.MOSTLY_Q5_0) and st.has_imatrix and i < n // 8:
        t = GT.Q4_1 if ftype == FT.MOSTLY_Q4_0 else GT.Q5_1
    st.i_ffn_down += 1
    return t


def _rule_attn_output(t: GT, ftype: FT, model: ModelInfo) -> GT:
    if model.arch == "falcon":
        return GT.Q4_K if ftype == FT.MOSTLY_Q3_K_L else t
    if model.n_expert == 8:
        if ftype in (FT.MOSTLY_Q2_K, FT.MOSTLY_IQ3_XS, FT.MOSTLY_IQ3_XXS, FT.MOSTLY_Q3_K_S,
                     FT.MOSTLY_Q3_K_M, FT.MOSTLY_IQ4_NL, FT.MOSTLY_Q4_K_S, FT.MOSTLY_Q4_K_M,
                     FT.MOSTLY_IQ3_S, FT.MOSTLY_IQ3_M, FT.MOSTLY_IQ4_XS):
            return GT.Q5_K
        return t
    return {FT.MOSTLY_Q2_K: GT.Q3_K, FT.MOSTLY_IQ3_XXS: GT.IQ3_S, FT.MOSTLY_Q3_K_M: GT.Q4_K,
            FT.MOSTLY_Q3_K_L: GT.Q5_K, FT.MOSTLY_IQ3_M: GT.Q4_K}.get(ftype, t)


def _rule_ffn_gate_up(st: QuantState, t: GT, ftype: FT, model: ModelInfo, name: str, up: bool) -> GT:
    counter = st.i_ffn_up if up else st.i_ffn_gate
    n = st.n_ffn_up if up else st.n_ffn_gate
    i, n = _layer(counter, n, name, model)
    if ftype == FT.MOSTLY_IQ3_XS and n // 8 <= i < 7 * n // 8:
        t = GT.IQ3_XXS
    if up:
        st.i_ffn_up += 1
    else:
        st.i_ffn_gate += 1
    return t


def _mixture(st: QuantState, model: ModelInfo, t: GT, name: str, ne: tuple[int, ...], ftype: FT,
             cat: Cat, emb_type: GT | None, out_type: GT | None) -> GT:
    ne2 = ne[2] if len(ne) > 2 else 1
    if cat == Cat.OUTPUT or (st.has_tied_embeddings and cat == Cat.TOKEN_EMBD):
        return _rule_output(t, ftype, model, ne[0], out_type)
    if ftype == FT.MOSTLY_MXFP4_MOE:
        return GT.MXFP4 if ne2 > 1 else GT.Q8_0
    if cat == Cat.TOKEN_EMBD:
        return _rule_token_embd(t, ftype, emb_type)
    if ftype in _IQ2_LIKE:
        return _rule_iq2_family(st, t, ftype, model, cat)
    if is_attn_v_like(cat):
        return _rule_attn_v(st, t, ftype, model)
    if cat == Cat.ATTN_K:
        if model.n_expert == 8:
            return GT.Q8_0
        return {FT.MOSTLY_IQ3_XS: GT.IQ3_XXS, FT.MOSTLY_IQ3_XXS: GT.IQ2_S}.get(ftype, t)
    if cat == Cat.ATTN_Q:
        return {FT.MOSTLY_IQ3_XS: GT.IQ3_XXS, FT.MOSTLY_IQ3_XXS: GT.IQ2_S}.get(ftype, t)
    if cat == Cat.FFN_DOWN:
        return _rule_ffn_down(st, t, ftype, model, name)
    if cat == Cat.ATTN_OUTPUT:
        return _rule_attn_output(t, ftype, model)
    if cat == Cat.ATTN_QKV:      # unreachable: attn_qkv is attn_v-like (kept for completeness)
        return t
    if cat in (Cat.FFN_GATE, Cat.FFN_UP):
        return _rule_ffn_gate_up(st, t, ftype, model, name, up=cat == Cat.FFN_UP)
    return t


def n_dims_of(ne: tuple[int, ...]) -> int:
    """ggml_n_dims: one past the highest axis with more than one element."""
    n = 1
    for i, d in enumerate(ne):
        if d > 1:
            n = i + 1
    return n


def tensor_get_type(st: QuantState, model: ModelInfo, name: str, ne: tuple[int, ...], src: GT,
                    ftype: FT, pure: bool = False, quantize_output_tensor: bool = True,
                    only_copy: bool = False, token_embedding_type: GT | None = None,
                    output_tensor_type: GT | None = None) -> GT:
    """Target type of one tensor (ne: ggml shape, ne[0] = row length); returns
    src for a tensor that stays as it is. Call in loader order."""
    if not allows_quantization(name, n_dims_of(ne), quantize_output_tensor, only_copy):
        return src
    cat = category(name)
    if token_embedding_type is not None and cat == Cat.TOKEN_EMBD:
        return token_embedding_type
    if output_tensor_type is not None and cat == Cat.OUTPUT:
        return output_tensor_type
    t = DEFAULT_TYPE.get(ftype)
    if t is None:
        raise ValueError(f"no default tensor type for ftype {ftype!r}")
    if not is_quantized(t):
        return t
    manual = next((ot for rx, ot in st.overrides if rx.search(name)), None)
    if manual is not None:
        t = manual
    elif not pure:
        t = _mixture(st, model, t, name, tuple(ne), ftype, cat, token_embedding_type,
                     output_tensor_type)
    return shape_fallback(st, name, ne[0], t)


def tensor_requires_imatrix(name: str, dst: GT, ftype: FT) -> bool:
    if name in _TOKEN_EMBD_NAMES or name == "output.weight":
        return False
    if dst in (GT.IQ3_XXS, GT.IQ2_XXS, GT.IQ2_XS, GT.IQ2_S, GT.IQ1_M, GT.IQ1_S):
        return True
    return dst == GT.Q2_K and ftype == FT.MOSTLY_Q2_K_S
