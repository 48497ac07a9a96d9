"""Run a program with libvkblas_hipblas.so interposed (LD_PRELOAD).

The reference is used as ``LD_PRELOAD=libvkblas_hipblas.so python script.py``
(reference README.md:56-70), and so is this library: the preloaded library
depends on no HIP runtime, and the engine it opens at the first GEMM binds to
the runtime the application loaded (PyTorch's bundled one, by soname).  On
gfx950 PyTorch's GEMMs go to hipBLASLt by default, whose hipblasLtMatmul this
library interposes (bias epilogues included); fp32 / fp16 / bf16 products
and linear layers therefore reach it with no change to the script.

This runner only builds that environment (this library ahead of whatever
the environment already preloads).  ``--torch-hipblas`` additionally makes
PyTorch use its hipBLAS backend instead of hipBLASLt (PyTorch then calls the
hipBLAS and rocBLAS entry points, as on the reference's gfx803), by making
``torch.backends.cuda.preferred_blas_library("cublas")`` before running an
unmodified Python script.

  python -m vkblas_amd.preload -- python my_script.py [args...]
  python -m vkblas_amd.preload --torch-hipblas -- python my_script.py [args...]
  python -m vkblas_amd.preload --torch-hipblas -- python -m my.module [args...]
"""
from __future__ import annotations

import os
import subprocess
import sys

from . import LIB_PATH


def preload_env(base: dict | None = None) -> dict:
    """Environment for a child process with the library preloaded (ahead of
    anything the environment already preloads, which stays)."""
    env = dict(os.environ if base is None else base)
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it first (make -C vkblas_amd)")
    old = env.get("LD_PRELOAD", "")
    env["LD_PRELOAD"] = ":".join([LIB_PATH] + ([old] if old else []))
    return env


# interpreter options that take a separate argument
_PY_OPTS_WITH_ARG = ("-W", "-X", "--check-hash-based-pycs")


def torch_hipblas_command(argv: list) -> list:
    """``python [opts] script.py args`` -> ``python [opts] -m vkblas_amd.torch_hipblas
    script.py args`` (``-m module`` in place of the script works the same);
    interpreter options such as ``-u`` stay with the interpreter."""
    i = 1
    while i < len(argv) and argv[i].startswith("-") and argv[i] not in ("-m", "-c", "-"):
        i += 2 if argv[i] in _PY_OPTS_WITH_ARG else 1
    if i >= len(argv) or argv[i] in ("-c", "-"):
        raise ValueError("--torch-hipblas needs: <python> [options] <script.py | -m module> [args...]")
    return argv[:i] + ["-m", "vkblas_amd.torch_hipblas"] + argv[i:]


def main(argv=None) -> int:
    argv = list(sys.argv[1:] if argv is None else argv)
    torch_hipblas = False
    if argv and argv[0] == "--torch-hipblas":
        torch_hipblas, argv = True, argv[1:]
    if argv and argv[0] == "--":
        argv = argv[1:]
    if not argv:
        print(__doc__, file=sys.stderr)
        return 2
    env = preload_env()
    if torch_hipblas:
        try:
            argv = torch_hipblas_command(argv)
        except ValueError as e:
            print(e, file=sys.stderr)
            return 2
        repo = os.path.dirname(os.path.dirname(LIB_PATH))
        env["PYTHONPATH"] = os.pathsep.join([repo] + ([env["PYTHONPATH"]] if env.get("PYTHONPATH") else []))
    return subprocess.call(argv, env=env)


if __name__ == "__main__":
    sys.exit(main())
