"""Build the gfx950 C-ABI library ``muspace_amd/native/libmuspace_msda.so``.

Replaces the reference's ``mcc`` + TVM-FFI AOT build
(/root/reference/native_build.py:27-65, sources listed in
/root/reference/build_utils.py:12-30) with one ``hipcc`` invocation over the
HIP sources in ``muspace_amd/csrc``. The library is built in-tree so that it
travels with the source tree; ``python -m muspace_amd.build`` rebuilds it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
SOURCES = (PACKAGE_DIR / "csrc" / "msda_capi.hip", PACKAGE_DIR / "csrc" / "dfa_capi.hip")
DEPENDS = (
    PACKAGE_DIR / "csrc" / "capi_errors.hpp",
    PACKAGE_DIR / "csrc" / "msda_device.hpp",
    PACKAGE_DIR / "csrc" / "msda_kernels.hpp",
    PACKAGE_DIR / "csrc" / "msda_backward_tiles.hpp",
    PACKAGE_DIR / "csrc" / "msda_forward_bin.hpp",
    PACKAGE_DIR / "csrc" / "dfa_kernels.hpp",
    REPO_DIR / "include" / "muspace_msda.h",
    REPO_DIR / "include" / "muspace_dfa.h",
)
LIBRARY = PACKAGE_DIR / "native" / "libmuspace_msda.so"
# memory-system probes for bench.py (--gather-probe, --atomic-probe); not
# loaded by the operators
PROBE_SOURCES = (PACKAGE_DIR / "csrc" / "probes.hip",)
PROBE_LIBRARY = PACKAGE_DIR / "native" / "libmuspace_probes.so"
OFFLOAD_ARCH = "gfx950"

# -packed-fp32-ops keeps the compiler from emitting packed fp32 VALU
# instructions (v_pk_*_f32); every kernel here is memory-bound, so nothing is
# lost.
HIPCC_FLAGS = (
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
)


def hipcc() -> str:
    found = shutil.which("hipcc")
    if found:
        return found
    fallback = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"
    if fallback.is_file():
        return str(fallback)
    raise FileNotFoundError("hipcc not found; ROCm is required to build libmuspace_msda.so")


def build_command(output: Path, sources=SOURCES) -> list[str]:
    return [hipcc(), *HIPCC_FLAGS, *(str(s) for s in sources), "-o", str(output)]


def _compile(library: Path, sources, verbose: bool) -> Path:
    library.parent.mkdir(parents=True, exist_ok=True)
    tmp = library.with_name(library.name + f".tmp{os.getpid()}")
    cmd = build_command(tmp, sources)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        tmp.unlink(missing_ok=True)
        raise RuntimeError(
            f"hipcc failed ({proc.returncode}) building {library.name}:\n{proc.stderr[-4000:]}"
        )
    os.replace(tmp, library)
    return library


def build(verbose: bool = False) -> Path:
    """Compile the MSDA library and the probe library (always), each moved
    into place atomically; returns the MSDA library's path."""
    _compile(PROBE_LIBRARY, PROBE_SOURCES, verbose)
    return _compile(LIBRARY, SOURCES, verbose)


def main(argv: list[str] | None = None) -> int:
    args = sys.argv[1:] if argv is None else argv
    path = build(verbose="-v" in args or "--verbose" in args)
    print(path)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
