"""Run a program with libvkblas_hipblas.so interposed on hipBLAS (LD_PRELOAD).

The reference is used as ``LD_PRELOAD=libvkblas_hipblas.so python script.py``
(reference README.md:56-70).  Under PyTorch-ROCm one more library has to lead
the preload list: torch ships its own HIP runtime (``torch/lib/libamdhip64.so``,
soname ``libamdhip64.so.7``) and loads it by the name ``libamdhip64.so``.  If
this library were preloaded alone it would pull in the system runtime
(``/opt/rocm/lib/libamdhip64.so.7``) first and the process would end up with
two HIP runtimes, whose streams and handles do not mix.  Preloading torch's
runtime first makes the library bind to that copy (matching soname), and
torch's later load of the same file is then a no-op.

hipBLAS must also be the BLAS backend PyTorch calls.  On gfx950 PyTorch's
default heuristic picks hipBLASLt, which this library does not intercept, and
no environment variable selects hipBLAS (``TORCH_BLAS_PREFER_HIPBLASLT`` can
only select hipBLASLt).  A script selects it with
``torch.backends.cuda.preferred_blas_library("cublas")``; ``--torch-hipblas``
runs an unmodified Python script with that call made first.

  python -m vkblas_amd.preload -- python my_script.py [args...]
  python -m vkblas_amd.preload --torch-hipblas -- python my_script.py [args...]
  python -m vkblas_amd.preload --torch-hipblas -- python -m my.module [args...]
"""
from __future__ import annotations

import os
import subprocess
import sys

from . import LIB_PATH


def torch_hip_runtime() -> str | None:
    """Path of the HIP runtime bundled with the installed torch, if any (found
    without importing torch, so no GPU is initialised here)."""
    import importlib.util
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.origin:
        return None
    path = os.path.join(os.path.dirname(spec.origin), "lib", "libamdhip64.so")
    return path if os.path.exists(path) else None


def preload_env(base: dict | None = None, with_torch_runtime: bool = True) -> dict:
    """Environment for a child process with the library preloaded."""
    env = dict(os.environ if base is None else base)
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it first (make -C vkblas_amd)")
    libs = []
    rt = torch_hip_runtime() if with_torch_runtime else None
    if rt:
        libs.append(rt)
    libs.append(LIB_PATH)
    old = env.get("LD_PRELOAD", "")
    env["LD_PRELOAD"] = ":".join(libs + ([old] if old else []))
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
