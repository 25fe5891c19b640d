"""Register and scratch use of the fused hard-network kernels (and of the
kernels that evaluate a conv block inside a conv network's head), read from the
gfx950 assembly (no GPU needed). A private (scratch) access in these
persistent kernels is a vector memory load that retires in order behind the
streamed input rows, so it stalls every layer: a spilled register or a
struct copied to scratch made the kernel several times slower. Every
instantiation must have no scratch instruction and no VGPR spill."""
import os
import re
import shutil
import subprocess

import pytest

from silogic_amd import _build

KERNEL = re.compile(
    r"^(_ZN3slg\d+(?:fc_hard_net_(?:rows|packed)|conv_head|conv_net)_kernel\w*):", re.M)


@pytest.fixture(scope="module")
def fc_hard_asm(tmp_path_factory):
    try:
        hipcc = _build._hipcc()
    except Exception as e:            # no ROCm toolchain on this host
        pytest.skip(str(e))
    if not shutil.which(hipcc) and not os.path.exists(hipcc):
        pytest.skip("hipcc not found")
    tmp = tmp_path_factory.mktemp("asm")
    procs = []
    for name in ("fc_hard", "conv_net"):
        src = os.path.join(_build.CSRC, name + ".hip")
        procs.append(subprocess.Popen(
            [hipcc] + _build.FLAGS + ["--cuda-device-only", "-S", "-I", _build.CSRC, src, "-o",
                                      str(tmp / (name + ".s"))],
            stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
    for p in procs:
        _, err = p.communicate()
        assert p.returncode == 0, err[-3000:]
    return (tmp / "fc_hard.s").read_text() + (tmp / "conv_net.s").read_text()


def test_fused_network_kernels_use_no_scratch(fc_hard_asm):
    text = fc_hard_asm
    names = KERNEL.findall(text)
    assert len(names) >= 32, len(names)
    assert sum("conv_head" in n for n in names) == 8, names
    assert sum("conv_net" in n for n in names) == 24, names
    bad = []
    for name in names:
        start = text.index(name + ":")
        body = text[start:text.index("s_endpgm", start)]
        if "scratch_" in body:
            bad.append((name, "scratch access"))
        meta = text[text.index(".name:           " + name):]
        spill = re.search(r"\.vgpr_spill_count:\s+(\d+)", meta)
        if spill and int(spill.group(1)):
            bad.append((name, "%s VGPR spills" % spill.group(1)))
    assert not bad, bad
