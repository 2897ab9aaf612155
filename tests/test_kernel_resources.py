"""Register and scratch budget of the hot kernels (CPU: compiles to gfx950
assembly with the library's own flags; no GPU).

The decode and prefill kernels are latency- or issue-bound, and two budgets
decide how they run:
- a kernel that spills to scratch memory needs a private segment per wave,
  and a spill in the verify window's gate/up launch made its time erratic
  (35 to 46 us per window between replays);
- the several-token gate/up launch must fit 128 registers so that four of
  its workgroups share a CU and its grid runs in one round.
"""
import concurrent.futures
import os
import re
import shutil
import subprocess
import tempfile

import pytest

from sager_amd import build_lib

# (source, kernel-name pattern, max private segment bytes, max VGPRs or None)
BUDGETS = [
    ("sg_layer.hip", r"layer_front_kernelILi1ELi8ELb1ELi1ELb[01]E", 0, None),
    ("sg_layer.hip", r"layer_front_kernelILi4ELi8ELb0ELi4ELb1E", 0, None),
    ("sg_layer.hip", r"layer_back_kernelILi2ELi8ELi[14]ELb[01]E", 0, None),
    ("sg_layer.hip", r"layer_gateup_kernelILi8ELi4ELb1E", 0, 128),
    ("sg_gemv.hip", r"gemv_lat_plain_kernel", 0, None),
    ("sg_gemv.hip", r"gemv1_kernelINS_9PlainRowsENS_6F32OutELi4E", 0, None),
    ("sg_prefill.hip", r"grouped_mfma_kernelILb[01]ELb[01]E", 0, None),
    ("sg_prefill.hip", r"route_quantize_kernel", 0, None),
    ("sg_q6.hip", r"gemv_q6_kernel", 0, None),
]


def _asm(src, out_dir):
    out = os.path.join(out_dir, src + ".s")
    flags = [f for f in build_lib.FLAGS if f not in ("-fPIC",)]
    cmd = [build_lib.HIPCC, *flags, "--cuda-device-only", "-S",
           os.path.join(build_lib.CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return src, open(out).read()


def _kernels(text):
    """name -> (private segment bytes, next free VGPR) from the kernel
    descriptors of a device assembly file."""
    res = {}
    for blk in text.split(".end_amdhsa_kernel")[:-1]:
        m = re.search(r"\.amdhsa_kernel (\S+)", blk)
        if not m:
            continue
        scratch = int(re.search(r"\.amdhsa_private_segment_fixed_size (\d+)", blk).group(1))
        vgpr = int(re.search(r"\.amdhsa_next_free_vgpr (\d+)", blk).group(1))
        res[m.group(1)] = (scratch, vgpr)
    return res


@pytest.mark.skipif(not os.path.exists(build_lib.HIPCC) and shutil.which("hipcc") is None,
                    reason="hipcc not available")
def test_hot_kernels_within_register_budget():
    srcs = sorted({s for s, *_ in BUDGETS})
    with tempfile.TemporaryDirectory() as d:
        with concurrent.futures.ThreadPoolExecutor(max_workers=len(srcs)) as ex:
            asm = dict(ex.map(lambda s: _asm(s, d), srcs))
    for src, pat, max_scratch, max_vgpr in BUDGETS:
        ks = {n: v for n, v in _kernels(asm[src]).items() if re.search(pat, n)}
        assert ks, f"no kernel matches {pat} in {src}"
        for name, (scratch, vgpr) in ks.items():
            assert scratch <= max_scratch, f"{name}: {scratch} B of scratch per lane"
            if max_vgpr is not None:
                assert vgpr <= max_vgpr, f"{name}: {vgpr} VGPRs (budget {max_vgpr})"
