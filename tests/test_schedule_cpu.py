"""Host-side checks of the attention forward's work schedule (csrc/flash_items.h), compiled with hipcc for
the host only and run without a GPU: every key tile of every item is covered once by its parts, padding
tiles once, split items' workspace slots are unique, and the kernel arguments fit in 4 KB."""

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


def _hipcc():
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    pytest.skip("hipcc not available")


def test_schedule_covers_every_tile_once(tmp_path):
    exe = tmp_path / "schedule_check"
    subprocess.run([_hipcc(), "-std=c++17", "-O1", f"-I{HERE.parent / 'include'}", str(HERE / "cpp" / "schedule_check.cpp"),
                    "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout
    # the shapes with few heads split items; the B*H = 16 ones do not
    lines = {l.split(":")[0]: l for l in r.stdout.splitlines()}
    assert "split items 0," not in lines["B=1 T=4096 H=2 causal=1 dense cus=256"]
    assert "split items 0," in lines["B=1 T=4096 H=16 causal=1 dense cus=256"]
    # a launch of one round folds its units; more than one round, a split launch or a ragged batch does not
    assert "fold 1," in lines["B=1 T=2048 H=16 causal=1 dense cus=256"]
    assert "fold 0," in lines["B=1 T=4096 H=16 causal=1 dense cus=256"]
    assert "fold 0," in lines["B=1 T=4096 H=2 causal=1 dense cus=256"]
    assert "fold 0," in lines["B=8 T=2048 H=16 causal=1 ragged cus=256"]
