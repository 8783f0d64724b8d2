"""Builds tests/cpp/dropin_check (host C++ only, g++) against include/ and libdirktensor_amd.so."""

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
BIN = HERE / "dropin_check"


def build() -> Path:
    libdir = ROOT / "dirktensor_amd"
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", f"-I{ROOT / 'include'}", str(HERE / "dropin_check.cpp"),
           "-o", str(BIN), f"-L{libdir}", "-ldirktensor_amd", f"-Wl,-rpath,{libdir}", "-Wl,-rpath,/opt/rocm/lib"]
    subprocess.run(cmd, check=True)
    return BIN


if __name__ == "__main__":
    print(build())
