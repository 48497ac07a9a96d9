"""Run a Python script or module with PyTorch's BLAS backend set to hipBLAS.

PyTorch-ROCm on gfx950 routes matmuls to hipBLASLt by default; the hipBLAS
entry points that libvkblas_hipblas.so interposes are only called once
``torch.backends.cuda.preferred_blas_library("cublas")`` is in effect.

  python -m vkblas_amd.torch_hipblas script.py [args...]
  python -m vkblas_amd.torch_hipblas -m package.module [args...]
"""
import runpy
import sys


def main() -> None:
    if len(sys.argv) < 2:
        print(__doc__, file=sys.stderr)
        sys.exit(2)
    import torch
    torch.backends.cuda.preferred_blas_library("cublas")
    if sys.argv[1] == "-m":
        if len(sys.argv) < 3:
            print(__doc__, file=sys.stderr)
            sys.exit(2)
        sys.argv = sys.argv[2:]
        runpy.run_module(sys.argv[0], run_name="__main__", alter_sys=True)
    else:
        sys.argv = sys.argv[1:]
        runpy.run_path(sys.argv[0], run_name="__main__")


if __name__ == "__main__":
    main()
