"""Build recipe for the oracle (test infrastructure, never the product).

* ``build_oracle()`` compiles ``oracle/ztcp_oracle.c`` (the CPU restatement)
  into ``oracle/build/libztcp_oracle.so``.
* ``build_ref()`` compiles the reference's own codec source,
  ``research/baseline_codec/csrc/fused_cold_page_cpu.cpp``, where it lies
  under /root/reference, into ``oracle/_ref/ztcp_fused_cold_page_cpp*.so``
  (a CPython extension, as the reference builds it with
  ``torch.utils.cpp_extension.load`` in native_fused_codec.py:58-64).  The
  flags are the reference's (``-O3 -std=c++17``) minus ``-march=armv8.5-a+fp16``
  (x86 g++ rejects it, so the portable scalar branches compile) and minus
  ``-ffast-math`` (parity target: strict IEEE fp32).  Nothing is copied: the
  compiler reads the file in place and writes only into ``oracle/_ref/``.

Run ``python oracle/build.py`` (both) or ``python oracle/build.py oracle``.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from pathlib import Path

HERE = Path(__file__).resolve().parent
REF_SRC = Path("/root/reference/research/baseline_codec/csrc/fused_cold_page_cpu.cpp")
REF_MODULE = "ztcp_fused_cold_page_cpp"


def build_oracle() -> Path:
    out_dir = HERE / "build"
    out_dir.mkdir(exist_ok=True)
    out = out_dir / "libztcp_oracle.so"
    cmd = [
        "gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off",
        "-fno-fast-math", "-Wall", "-Wextra", "-Wno-unused-parameter",
        str(HERE / "ztcp_oracle.c"), "-o", str(out), "-lm", "-lpthread",
    ]
    subprocess.run(cmd, check=True)
    return out


def ref_available() -> bool:
    return REF_SRC.is_file()


def build_ref() -> Path | None:
    """Compile the reference codec; returns None when the reference is absent."""
    if not ref_available():
        return None
    import torch.utils.cpp_extension as ce

    out_dir = HERE / "_ref"
    out_dir.mkdir(exist_ok=True)
    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = out_dir / f"{REF_MODULE}{suffix}"
    incs = [f"-I{p}" for p in ce.include_paths()] + [f"-I{sysconfig.get_paths()['include']}"]
    libdirs = ce.library_paths()
    import torch

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = (
        ["g++", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
         f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
         f"-DTORCH_EXTENSION_NAME={REF_MODULE}", "-DTORCH_API_INCLUDE_EXTENSION_H",
         "-w"]
        + incs
        + [str(REF_SRC), "-o", str(out)]
        + [f"-L{d}" for d in libdirs]
        + [f"-Wl,-rpath,{d}" for d in libdirs]
        + ["-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"]
    )
    subprocess.run(cmd, check=True)
    return out


if __name__ == "__main__":
    what = sys.argv[1:] or ["oracle", "ref"]
    if "oracle" in what:
        print(build_oracle())
    if "ref" in what:
        print(build_ref())
