"""CPU: every gfx950 kernel of the library compiles without register spills.

A kernel that spills keeps part of its state in scratch memory: every such access is an HBM
round trip (a 48-byte struct spilled in the accept decision once cost a write of ~3 KB per
block and a dependent read).  The build's own flags, device code only, with the compiler's
per-kernel resource report; skipped where hipcc is absent.
"""
import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

from iitj_llm_coopt_amd import build as B

HIPCC = next((c for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc"))
              if c and os.path.exists(c)), None)


def resources(src, tmp):
    cmd = [HIPCC, *B.HIP_FLAGS, "--cuda-device-only", "-S", "-Rpass-analysis=kernel-resource-usage",
           os.path.join(B.CSRC, src), "-o", os.path.join(tmp, src + ".s")]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    out, name = {}, None
    for line in res.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name:
            out[name] = int(m.group(1))
    return out


@pytest.mark.skipif(HIPCC is None, reason="hipcc not installed")
def test_no_kernel_spills_to_scratch(tmp_path):
    with ThreadPoolExecutor(len(B.SOURCES)) as ex:
        per_file = dict(zip(B.SOURCES, ex.map(lambda s: resources(s, str(tmp_path)), B.SOURCES)))
    kernels = {f"{src}:{k}": v for src, ks in per_file.items() for k, v in ks.items()}
    assert len(kernels) > 20, kernels  # the report was parsed
    spilled = {k: v for k, v in kernels.items() if v}
    assert not spilled, f"kernels using scratch (bytes/lane): {spilled}"
