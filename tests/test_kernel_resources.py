"""Register-spill and occupancy guards for the hot kernels (CPU only: compiles, runs nothing).

The cache-latent prefill and the paged decode share `mqa_fwd_kernel`.  Scratch traffic inside
its tile loop costs every tile, and outside it a spill reload is followed by a `vmcnt` wait
that drains the copies and stores in flight (on gfx9 loads and stores share that counter).
This test compiles csrc/dmla_fwd.hip for gfx950 with the Makefile's flags and checks, in both
instantiations, that
  * no basic block that issues MFMAs (the tile iterations) touches scratch, and
  * the scratch accesses that remain sit next to the call of the overflow (exact-max) path,
    which the normal path never takes -- apart from at most four per kernel (decode keeps one
    64-bit value in scratch across its segment loop: one store, one reload per instantiation).
"""
import os
import re
import subprocess

import pytest

from conftest import ROOT

CSRC = os.path.join(ROOT, "ds-flashdmla-moe_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-I" + os.path.join(ROOT, "include"),
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form",
         "-Wno-unused-function", "--cuda-device-only", "-S"]


def _blocks(body):
    """Splits a function's assembly into basic blocks (labels and %bb comments start one)."""
    blocks, cur = [], []
    for line in body:
        if re.match(r"^(\.LBB\d+_\d+:|; %bb\.\d+:)", line):
            if cur:
                blocks.append(cur)
            cur = [line]
        else:
            cur.append(line)
    if cur:
        blocks.append(cur)
    return blocks


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is needed")
def test_forward_tile_loops_are_spill_free(tmp_path):
    out = tmp_path / "fwd.s"
    run = subprocess.run([HIPCC] + FLAGS + [os.path.join(CSRC, "dmla_fwd.hip"), "-o", str(out)],
                         capture_output=True, text=True, timeout=600)
    assert run.returncode == 0, run.stderr[-2000:]
    asm = out.read_text()
    for decode in (0, 1):
        name = f"_ZN4dmla12_GLOBAL__N_114mqa_fwd_kernelILb{decode}EEEvNS0_9MqaParamsE:"
        start = asm.index(name)
        body = asm[start:asm.index(".Lfunc_end", start)].split("\n")
        ins = [l.strip() for l in body]
        calls = [i for i, l in enumerate(ins) if l.startswith("s_swappc")]
        assert calls, "the exact-path call is expected in the kernel"
        for blk in _blocks(body):
            lines = [l.strip() for l in blk]
            mfma = sum(1 for l in lines if l.startswith("v_mfma"))
            scratch = [l for l in lines if l.startswith("scratch_")]
            if mfma >= 16 and not any(l.startswith("s_swappc") for l in lines):
                assert not scratch, f"kernel {decode}: scratch access in a tile iteration: {scratch[:2]}"
        far = [i for i, l in enumerate(ins) if l.startswith("scratch_") and all(abs(i - c) > 40 for c in calls)]
        assert len(far) <= 4, f"kernel {decode}: {len(far)} scratch accesses outside the exact-path call"


# Occupancy each backward kernel's tuning assumes (waves per SIMD the compiler reports for it):
# the on-the-fly dQ kernel runs three workgroups per CU (a third wave per SIMD covers more of
# its sub-tiles' dependent chain), the others two, and the cache-latent dK/dV kernel one wave
# per SIMD with its 512 registers.  None of them may spill.
_BWD_OCCUPANCY = {
    "dmla_bwd.hip": {"bwd_dkdv_kernel": 1, "bwd_dq_kernel": 2},
    "dmla_otf_bwd.hip": {"otf_bwd_dkdv_kernel": 2, "otf_bwd_dq_kernel": 3, "otf_bwd_wgrad_kernel": 2},
}


def _kernel_stats(asm):
    """kernel short name -> (VGPRs, scratch bytes, occupancy) from the compiler's comments."""
    stats = {}
    for m in re.finditer(r"^_ZN4dmla\S*?((?:otf_)?bwd_[a-z_]+?_kernel)\S*:", asm, re.M):
        rest = asm[m.end():]
        get = lambda key: int(re.search(r"; %s: (\d+)" % key, rest).group(1))
        stats[m.group(1)] = (get("NumVgprs"), get("ScratchSize"), get("Occupancy"))
    return stats


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is needed")
@pytest.mark.parametrize("source", sorted(_BWD_OCCUPANCY))
def test_backward_kernels_keep_occupancy_without_spills(tmp_path, source):
    out = tmp_path / (source + ".s")
    run = subprocess.run([HIPCC] + FLAGS + [os.path.join(CSRC, source), "-o", str(out)],
                         capture_output=True, text=True, timeout=600)
    assert run.returncode == 0, run.stderr[-2000:]
    stats = _kernel_stats(out.read_text())
    for name, (vgprs, scratch, occupancy) in stats.items():
        assert scratch == 0, f"{name}: {scratch} bytes of scratch ({vgprs} VGPRs)"
    for name, want in _BWD_OCCUPANCY[source].items():
        assert name in stats, f"{name} not found in {source}"
        assert stats[name][2] >= want, f"{name}: occupancy {stats[name][2]} < {want} ({stats[name][0]} VGPRs)"
