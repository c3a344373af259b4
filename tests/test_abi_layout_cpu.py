"""CPU-side: the ctypes mirrors in pulsatrix_amd/native.py have the C layout of include/pxk.h and
include/pulsatrix_amd.h.

A mirror shorter than the C struct, or with a field at another offset, would hand the kernels
whatever bytes follow it as pointers. A small C program compiled against the header prints each
struct's size and every field's offset, and they must equal ctypes' view of the mirror.
"""
import ctypes
import os
import subprocess
import tempfile

import pytest

from pulsatrix_amd import native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MIRRORS = [("pxk_gemm_desc", N.GemmDesc), ("pxk_operand", N.Operand), ("pxk_attn_rel_desc", N.AttnRelDesc),
           ("pxk_attn_rel_kv_desc", N.AttnRelKvDesc), ("pxk_rule_params", N.RuleParams),
           ("pxk_rule_block", N.RuleBlock), ("px_model_config", N.ModelConfig), ("px_lrp_rule", N.LrpRule)]


def c_layout(struct, fields):
    src = ['#include <stddef.h>', '#include <stdio.h>', '#include "pxk.h"', '#include "pulsatrix_amd.h"',
           "int main(void) {",
           '  printf("size %%zu\\n", sizeof(%s));' % struct]
    src += ['  printf("%s %%zu\\n", offsetof(%s, %s));' % (f, struct, f) for f in fields]
    src += ["  return 0;", "}"]
    with tempfile.TemporaryDirectory() as tmp:
        c = os.path.join(tmp, "layout.c")
        exe = os.path.join(tmp, "layout")
        open(c, "w").write("\n".join(src) + "\n")
        subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), c, "-o", exe], check=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    return {k: int(v) for k, v in (line.split() for line in out.splitlines())}


@pytest.mark.parametrize("struct,mirror", MIRRORS)
def test_ctypes_mirror_matches_c_layout(struct, mirror):
    fields = [f for f, _ in mirror._fields_]
    want = c_layout(struct, fields)
    assert ctypes.sizeof(mirror) == want["size"]
    for f in fields:
        assert getattr(mirror, f).offset == want[f], f
