"""Build helpers (hip_kernels/build_utils.py:34-298 of the reference).

The reference compiles its HIP source at first use into ~/.cache.  This
package's library is compiled ahead of time for gfx950
(rocm-qlora_amd/build.py) and only loaded at run time; these helpers locate
hipcc, compile a standalone .hip file, and report the prebuilt library.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from typing import Optional

HIP_FLAGS = ["-O3", "-fPIC", "-shared", "-std=c++17",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def find_hipcc() -> Optional[str]:
    """Path of hipcc ($HIPCC, PATH, then $ROCM_PATH/bin), or None."""
    env = os.environ.get("HIPCC")
    if env and os.path.isfile(env):
        return env
    found = shutil.which("hipcc")
    if found:
        return found
    cand = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")
    return cand if os.path.isfile(cand) else None


def is_hipcc_available() -> bool:
    return find_hipcc() is not None


def compile_hip_kernel(src_path: str, out_path: str, arch: str = "gfx950", timeout: int = 300) -> bool:
    """Compile one .hip file into a shared library; False on any failure."""
    hipcc = find_hipcc()
    if hipcc is None or not os.path.isfile(src_path):
        return False
    os.makedirs(os.path.dirname(os.path.abspath(out_path)), exist_ok=True)
    cmd = [hipcc, f"--offload-arch={arch}", *HIP_FLAGS, src_path, "-o", out_path]
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
    except (OSError, subprocess.TimeoutExpired):
        return False
    return r.returncode == 0 and os.path.isfile(out_path)


def get_or_compile_int4_kernel() -> Optional[str]:
    """Path of the prebuilt librocm_qlora_amd.so, or None when it has not
    been built.  Nothing is compiled here."""
    from rocm_qlora import _native
    return _native.LIB_PATH if os.path.isfile(_native.LIB_PATH) else None
