"""CPU check of the page-major Key scale/min layout helpers shared by the packers and the decode
kernel (logitfill_amd/csrc/lf_common.hpp: sm_page, sm_slot, sm_place): tests/sm_page_check.cpp,
compiled from the real header, checks for every tier width that sm_place inverts sm_slot, that
no two ranks share a position and that positions stay inside the tier's blocks; the Python
mirror of the block count (packed.layout.sm_page_elems, which sizes the buffers) agrees with the
C one."""
import shutil
import subprocess
from pathlib import Path

import pytest

from logitfill_amd.packed.layout import sm_page_elems

ROOT = Path(__file__).resolve().parents[1]
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="needs hipcc")
def test_sm_place_inverts_sm_slot(tmp_path):
    exe = tmp_path / "sm_page_check"
    subprocess.run([HIPCC, "-x", "hip", "--offload-arch=gfx950", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "sm_page_check.cpp"), "-o", str(exe)], check=True, capture_output=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr


def test_block_count_known_answers():
    # c2's seed-0 mix at Key 3.0 bits: words (7, 4, 3) -> K-steps 4 + 1 + 1 = 6, 24 blocks
    assert sm_page_elems((7, 4, 3)) == 16 * 24
    # one int2 word: 2 K-steps (a K-step takes half of 4 words); one int8 word: 1 K-step
    assert sm_page_elems((1, 0, 0)) == 16 * 8
    assert sm_page_elems((0, 0, 1)) == 16 * 4
    assert sm_page_elems((8, 16, 32)) == 16 * 4 * (4 + 4 + 4)
    assert sm_page_elems((0, 0, 0)) == 0
