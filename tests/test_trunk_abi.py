"""The plugin's Ds4fGpuTrunkTensor has the layout of the engine's
Ds4fTrunkTensor (include/ds4f/moe.h:49-56), so the engine can pass its parsed
tensor list (tl->t + tl->t_off[L]) to ds4f_gpu_attn_weights_trunk by a
pointer cast.  This compiles a translation unit holding both headers with
static assertions on the size, the alignment and every field's offset and
size; it needs the reference's headers and is skipped where they are absent
(no GPU)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INC = "/root/reference/include"

FIELDS = ["name", "dtype", "dims", "rank", "off", "nbytes"]


@pytest.mark.skipif(not os.path.exists(os.path.join(REF_INC, "ds4f", "moe.h")),
                    reason="the reference's headers are not present")
@pytest.mark.skipif(shutil.which("gcc") is None, reason="no C compiler")
def test_trunk_tensor_layout_matches_reference(tmp_path):
    lines = ['#include <stddef.h>', '#include "ds4f/moe.h"', '#include "ds4f_gpu_attn.h"',
             "#define SAME(expr, what) _Static_assert(expr, what)",
             "SAME(sizeof(Ds4fGpuTrunkTensor) == sizeof(Ds4fTrunkTensor), \"size\");",
             "SAME(_Alignof(Ds4fGpuTrunkTensor) == _Alignof(Ds4fTrunkTensor), \"alignment\");"]
    for f in FIELDS:
        lines.append(f"SAME(offsetof(Ds4fGpuTrunkTensor, {f}) == offsetof(Ds4fTrunkTensor, {f}), "
                     f"\"offset of {f}\");")
        lines.append(f"SAME(sizeof(((Ds4fGpuTrunkTensor *)0)->{f}) == "
                     f"sizeof(((Ds4fTrunkTensor *)0)->{f}), \"size of {f}\");")
    # a planted mismatch must fail the same way, so the check can fail at all
    bad = lines[:3] + ["typedef struct { char name[96]; int dtype; int dims[4]; int rank; "
                       "long off; long nbytes; } Wrong;",
                       "_Static_assert(offsetof(Wrong, rank) == offsetof(Ds4fTrunkTensor, rank), "
                       "\"planted\");"]
    for body, ok in (("\n".join(lines), True), ("\n".join(bad), False)):
        src = tmp_path / "abi.c"
        src.write_text(body + "\n")
        r = subprocess.run(["gcc", "-std=c11", "-fsyntax-only", "-I", REF_INC,
                            "-I", os.path.join(ROOT, "include"), str(src)],
                           capture_output=True, text=True)
        assert (r.returncode == 0) == ok, r.stderr
