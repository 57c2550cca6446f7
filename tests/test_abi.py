"""CPU checks of the C ABI: header <-> library exports, struct layouts."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

from conftest import REPO

HEADER = os.path.join(REPO, "include", "dgm_quant.h")


def header_functions():
    text = open(HEADER).read()
    return set(re.findall(r"^\s*(?:int64_t|int|void\s*\*?|const char\s*\*)\s*(dgm_\w+)\s*\(", text, re.M))


def test_header_declares_the_reference_surface():
    names = header_functions()
    # Kernel-level entries (metal/kernels.metal) and GPU.swift wrappers.
    for n in ["dgm_quant_i8", "dgm_quant_i4", "dgm_gemm_nt_f32", "dgm_gemm_nt_i8", "dgm_gemm_nt_i4",
              "dgm_gemm_dx_f32", "dgm_gemm_dx_i8", "dgm_gemm_dx_i4", "dgm_gemm_dw", "dgm_gemm_dw_acc",
              "dgm_quantize", "dgm_gemmNT", "dgm_gemmDX", "dgm_gemmDW", "dgm_gemmDWAcc",
              "dgm_begin", "dgm_end", "dgm_last_kernel",
              # the DiT loop body's wrappers (src/GPU.swift:211-410) and the block forward
              "dgm_rmsFwd", "dgm_ropeFwd", "dgm_repeatHeads", "dgm_attnFwd", "dgm_swigluFwd", "dgm_add",
              "dgm_mix", "dgm_copy", "dgm_ropeTables", "dgm_dit_forward", "dgm_dit_workspace_floats"]:
        assert n in names


def test_library_exports_every_declared_symbol(dgm):
    lib = dgm.load_library()
    names = header_functions()
    assert names == set(dgm.PROTOTYPES), "binding prototypes drifted from the header"
    for n in names:
        assert hasattr(lib, n), n


def test_param_block_layouts_compile(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(
        '#include "dgm_quant.h"\n#include <stddef.h>\n'
        "_Static_assert(sizeof(dgm_GemmP) == 32, \"GemmP\");\n"
        "_Static_assert(sizeof(dgm_QuantP) == 16, \"QuantP\");\n"
        "_Static_assert(offsetof(dgm_GemmP, qGroup) == 16, \"qGroup\");\n"
        "_Static_assert(offsetof(dgm_QuantP, qmax) == 8, \"qmax\");\n"
        "int main(void) { return 0; }\n")
    subprocess.run(["gcc", "-std=c11", "-fsyntax-only", "-I", os.path.join(REPO, "include"), str(src)],
                   check=True)
    from dgm_amd import GemmP, QuantP
    assert ctypes.sizeof(GemmP) == 32 and ctypes.sizeof(QuantP) == 16
    assert QuantP.qmax.offset == 8 and GemmP.qGroup.offset == 16


def test_product_does_not_touch_the_oracle():
    """The shipped package never imports, links or calls the CPU oracle."""
    pkg = os.path.join(REPO, "diffusion-gpt-metal_amd")
    banned = re.compile(r"import\s+oracle|from\s+oracle|liboracle|\borc_\w+\(")
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp", ".h")):
                text = open(os.path.join(root, f), errors="ignore").read()
                assert not banned.search(text), f


def test_workspace_bound_closed_forms(dgm):
    """dgm_gemmNT_workspace_bound is host arithmetic: the decode pieces'
    260 K + 512 bytes, the K-sliced partial sums (M <= 16, at most K / 256
    slices, capped at the static scratch), the bf16 copy of X above 64 rows."""
    lib = dgm.load_library()
    f = lib.dgm_gemmNT_workspace_bound
    assert f(1, 14336, 4096) == 260 * 4096 + 512                  # partials 917,504 < pieces
    assert f(16, 14336, 4096) == dgm.DGM_NOALLOC_SCRATCH_BYTES     # 14.7 MB of partials, capped
    assert f(8, 1024, 4096) == max(260 * 4096 + 512, 8 * 1024 * 16 * 4)
    assert f(64, 14336, 4096) == 260 * 4096 + 512
    assert f(8192, 14336, 4096) == 2 * 8192 * 4096
    assert f(65, 10, 100) == 260 * 100 + 512                       # 2 M K = 13,000 is smaller
    assert f(0, 0, 0) == 512
    assert f(-1, 4, 4) == -1 and f(4, -1, 4) == -1 and f(4, 4, -1) == -1
