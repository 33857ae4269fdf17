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
    # the device's initialisation starts first, on a thread of its own; the
    # command line's imports, parsing and planning then overlap it
    early = importlib.import_module("quant-studio_amd.pipeline_start").early_start(sys.argv[1:])
    try:
        cli = importlib.import_module("quant-studio_amd.cli")
    except BaseException:
        if early is not None:
            early.close()
        raise
    sys.exit(cli.main(early=early))
