"""CPU checks of the compiled kernels' resources (no GPU): the hot kernels of
the block keep every value in registers.

A register spill on gfx950 goes to scratch, which lives in device memory:
each spilled lane stores and reloads its values through the caches to HBM.
The offset-free flash pass once spilled 84 bytes a lane (the 64-bit query
indices of its Q loads, kept across the key loop for the output stores), and
over the 2.1 M lanes of one N = 1024 launch that was 0.17 GB of writes and as
much fetch on top of the 0.27 GB of output. These tests compile the kernel
sources to gfx950 assembly with the build's own flags and read the resource
metadata the compiler emits for each kernel."""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from foldjax_amd import build as B

# (source file, kernel symbol fragment): the kernels a Pairformer block at the
# headline configuration spends its time in
HOT = [
    ("fjx_flash_pipe.hip", "flash_pipe_kernel_bf16"),
    ("fjx_contract.hip", "contract_dma_kernel"),
    ("fjx_rowproj.hip", "trimul_prologue_kernel"),
    ("fjx_rowproj.hip", "trimul_epilogue_kernel"),
    ("fjx_rowproj.hip", "triattn_prologue_kernel"),
    ("fjx_rowproj.hip", "triattn_epilogue_kernel"),
    ("fjx_transition.hip", "transition128_pbf32_kernel"),
    ("fjx_transition.hip", "transition128_kernel"),
]


def _kernel_metadata(src: str, tmp_path: Path) -> dict[str, dict[str, int]]:
    hipcc = B._hipcc()
    if not shutil.which(hipcc) and not Path(hipcc).is_file():
        pytest.skip("hipcc is not available")
    out = tmp_path / (Path(src).stem + ".s")
    cmd = [hipcc, *B.HIP_FLAGS, *B.FILE_FLAGS.get(src, []), "--cuda-device-only", "-S", str(B.CSRC / src), "-o",
           str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    meta: dict[str, dict[str, int]] = {}
    name = None
    for line in out.read_text().splitlines():
        m = re.match(r"\s*\.name:\s+(\S+)", line)
        if m:
            name = m.group(1)
            meta[name] = {}
            continue
        m = re.match(r"\s*\.(private_segment_fixed_size|vgpr_spill_count|sgpr_spill_count|vgpr_count):\s+(\d+)", line)
        if m and name is not None:
            meta[name][m.group(1)] = int(m.group(2))
    return meta


@pytest.fixture(scope="module")
def metadata(tmp_path_factory):
    tmp = tmp_path_factory.mktemp("isa")
    return {src: _kernel_metadata(src, tmp) for src in sorted({s for s, _ in HOT})}


@pytest.mark.parametrize("src,kernel", HOT)
def test_hot_kernel_does_not_spill(metadata, src, kernel):
    found = {n: m for n, m in metadata[src].items() if kernel in n}
    assert found, f"{kernel} not found in {src}"
    for name, m in found.items():
        assert m.get("private_segment_fixed_size", 0) == 0, f"{name} uses {m} bytes of scratch"
        assert m.get("vgpr_spill_count", 0) == 0, f"{name} spills: {m}"


def test_flash_pass_keeps_two_waves_per_simd(metadata):
    # 512 registers per SIMD lane: two waves need at most 256 each
    for name, m in metadata["fjx_flash_pipe.hip"].items():
        if "flash_pipe_kernel_bf16" in name:
            assert m["vgpr_count"] <= 256, (name, m)
