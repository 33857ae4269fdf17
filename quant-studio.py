#!/usr/bin/env python3
"""quant-studio: GGUF -> GGUF quantization on AMD Instinct MI355X.

    python quant-studio.py in.gguf out.gguf Q4_K_M --imatrix imatrix.gguf --mem 4G

Drop-in for the reference's quant-studio.py command line; the implementation is
the quant-studio_amd package (HIP kernels through a C ABI).
"""

import importlib
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent))

if __name__ == "__main__":
    sys.exit(importlib.import_module("quant-studio_amd.cli").main())
