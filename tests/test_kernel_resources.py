"""Every device kernel of the library fits its registers: no scratch (private
segment) use.  A spill costs far more than the registers it saves on these
bandwidth-bound kernels (an 8-byte spill in the MoE down-projection kernel
made the top-10 gather 40% slower), so a kernel that starts to spill after a
change fails here instead of showing up only as a slower benchmark.

Compiles each csrc/*.hip for gfx950 to assembly with the library's own flags
(about 25 s on 8 cores) and reads the per-kernel private segment size."""

import concurrent.futures as cf
import re
import shutil
import subprocess

import pytest

from gdsllm_amd import build as b

SOURCES = sorted(b.CSRC.glob("*.hip"))


def _device_asm(src, out_dir):
    out = out_dir / (src.stem + ".s")
    cmd = [b.hipcc(), *b.HIPCC_FLAGS, "--cuda-device-only", "-S", "-o", str(out), str(src)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, f"{src.name}: {res.stderr[-2000:]}"
    return out.read_text()


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    if shutil.which("hipcc") is None and not (b.Path(b.ROCM) / "bin" / "hipcc").exists():
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("asm")
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        texts = list(ex.map(lambda s: _device_asm(s, d), SOURCES))
    return dict(zip((s.name for s in SOURCES), texts))


def test_no_kernel_uses_scratch(device_asm):
    spills = []
    kernels = 0
    for name, text in device_asm.items():
        for m in re.finditer(r"\.set\s+(\S+)\.private_seg_size,\s*(\d+)", text):
            kernels += 1
            if int(m.group(2)) != 0:
                spills.append(f"{name}: {m.group(1)} ({m.group(2)} bytes)")
    assert kernels > 50, f"found only {kernels} kernels in the assembly"
    assert not spills, "kernels with scratch:\n" + "\n".join(spills)
