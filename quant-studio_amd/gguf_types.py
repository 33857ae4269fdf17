"""GGUF enum values used by the quantizer registry (public GGUF spec values).

The reference takes these from gguf-py (kernels/common.py:6-7); gguf-py is not
a dependency here, so the ids are restated.
"""

from __future__ import annotations

import enum


class GGMLQuantizationType(enum.IntEnum):
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    IQ2_XXS = 16
    IQ2_XS = 17
    IQ3_XXS = 18
    IQ1_S = 19
    IQ4_NL = 20
    IQ3_S = 21
    IQ2_S = 22
    IQ4_XS = 23
    I8 = 24
    I16 = 25
    I32 = 26
    I64 = 27
    F64 = 28
    IQ1_M = 29
    BF16 = 30
    TQ1_0 = 34
    TQ2_0 = 35
    MXFP4 = 39
    # named by the scheme table only; not in the public type table this build
    # restates, so they get ids outside it
    Q1_0 = 100
    Q2_0 = 101


class LlamaFileType(enum.IntEnum):
    ALL_F32 = 0
    MOSTLY_F16 = 1
    MOSTLY_Q4_0 = 2
    MOSTLY_Q4_1 = 3
    MOSTLY_Q8_0 = 7
    MOSTLY_Q5_0 = 8
    MOSTLY_Q5_1 = 9
    MOSTLY_Q2_K = 10
    MOSTLY_Q3_K_S = 11
    MOSTLY_Q3_K_M = 12
    MOSTLY_Q3_K_L = 13
    MOSTLY_Q4_K_S = 14
    MOSTLY_Q4_K_M = 15
    MOSTLY_Q5_K_S = 16
    MOSTLY_Q5_K_M = 17
    MOSTLY_Q6_K = 18
    MOSTLY_IQ2_XXS = 19
    MOSTLY_IQ2_XS = 20
    MOSTLY_Q2_K_S = 21
    MOSTLY_IQ3_XS = 22
    MOSTLY_IQ3_XXS = 23
    MOSTLY_IQ1_S = 24
    MOSTLY_IQ4_NL = 25
    MOSTLY_IQ3_S = 26
    MOSTLY_IQ3_M = 27
    MOSTLY_IQ2_S = 28
    MOSTLY_IQ2_M = 29
    MOSTLY_IQ4_XS = 30
    MOSTLY_IQ1_M = 31
    MOSTLY_BF16 = 32
    MOSTLY_TQ1_0 = 36
    MOSTLY_TQ2_0 = 37
    MOSTLY_MXFP4_MOE = 38
    MOSTLY_Q1_0 = 100
    MOSTLY_Q2_0 = 101


_T = GGMLQuantizationType
# (values per block, bytes per block): the public GGML type table
QUANT_SIZES: dict[GGMLQuantizationType, tuple[int, int]] = {
    _T.F32: (1, 4), _T.F16: (1, 2), _T.Q4_0: (32, 18), _T.Q4_1: (32, 20), _T.Q5_0: (32, 22),
    _T.Q5_1: (32, 24), _T.Q8_0: (32, 34), _T.Q8_1: (32, 36), _T.Q2_K: (256, 84),
    _T.Q3_K: (256, 110), _T.Q4_K: (256, 144), _T.Q5_K: (256, 176), _T.Q6_K: (256, 210),
    _T.Q8_K: (256, 292), _T.IQ2_XXS: (256, 66), _T.IQ2_XS: (256, 74), _T.IQ3_XXS: (256, 98),
    _T.IQ1_S: (256, 50), _T.IQ4_NL: (32, 18), _T.IQ3_S: (256, 110), _T.IQ2_S: (256, 82),
    _T.IQ4_XS: (256, 136), _T.I8: (1, 1), _T.I16: (1, 2), _T.I32: (1, 4), _T.I64: (1, 8),
    _T.F64: (1, 8), _T.IQ1_M: (256, 56), _T.BF16: (1, 2), _T.TQ1_0: (256, 54),
    _T.TQ2_0: (256, 66), _T.MXFP4: (32, 17), _T.Q1_0: (128, 18), _T.Q2_0: (64, 18),
}
