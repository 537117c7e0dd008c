"""Register budget of every HIP kernel (CPU only: compiles the sources to
gfx950 assembly with the library's own flags). A kernel that spills VGPRs or
uses scratch memory reloads through the vector memory path and waits on
vmcnt behind its own streaming loads; this guards against that regression
(head_dim 256 decode once spilled 118 registers and ran at half speed)."""
import concurrent.futures as cf
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from runtherder_amd import build as B

HIP_SOURCES = [s for s in B.KERNEL_SOURCES if s.endswith(".hip")]


def _assemble(src: str, out_dir: Path) -> str:
    out = out_dir / (Path(src).stem + ".s")
    flags = [f for f in B.DEVICE_FLAGS if f != "-fPIC"]
    cmd = [B.HIPCC, *flags, "-x", "hip", "--cuda-device-only", "-S", str(B.CSRC / src),
           "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def _kernels(asm: str) -> dict[str, dict[str, int]]:
    """Per-kernel .private_segment_fixed_size / .vgpr_spill_count /
    .sgpr_spill_count from the code object metadata."""
    res: dict[str, dict[str, int]] = {}
    for block in re.split(r"\n\s+- \.", asm.split("amdhsa.kernels:", 1)[-1]):
        name = re.search(r"\.name:\s+(\S+)", block)
        if not name:
            continue
        vals = {k: int(v) for k, v in re.findall(
            r"\.(private_segment_fixed_size|vgpr_spill_count|sgpr_spill_count):\s+(\d+)", block)}
        res[name.group(1)] = vals
    return res


@pytest.mark.skipif(shutil.which(B.HIPCC) is None and not Path(B.HIPCC).exists(),
                    reason="hipcc not available")
def test_no_kernel_spills_or_scratch(tmp_path):
    with cf.ThreadPoolExecutor(max_workers=len(HIP_SOURCES)) as ex:
        asms = dict(zip(HIP_SOURCES, ex.map(lambda s: _assemble(s, tmp_path), HIP_SOURCES)))
    bad = []
    n = 0
    for src, asm in asms.items():
        for name, vals in _kernels(asm).items():
            n += 1
            # SGPR spills land in VGPR lanes (v_writelane / v_readlane), not in
            # memory, so only VGPR spills and scratch count.
            if any(vals.get(k, 0) for k in ("private_segment_fixed_size", "vgpr_spill_count")):
                bad.append((src, name[:90], vals))
    assert n >= 50, f"parsed only {n} kernels"
    assert not bad, bad
