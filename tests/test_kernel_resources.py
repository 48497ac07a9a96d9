"""Register spills of the built gfx950 kernels, read from the code objects'
own AMDGPU metadata (.vgpr_spill_count, .private_segment_fixed_size) in
libvkblas_engine.so: no kernel may spill to scratch memory, which costs
scratch writes on every call (the pipelined GEMM kernels once wrote up to
6 MiB of spills per 8192^3 fp16 call).  One documented exception: the
unsplit four-activation-tile form of the 16-bit K x N decode kernel spills
28 VGPRs in its epilogue, after its K loop.  CPU only: the LLVM tools of the
ROCm install unbundle the code objects."""
import os
import re
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ENGINE = os.path.join(HERE, "..", "vkblas_amd", "libvkblas_engine.so")
LLVM = "/opt/rocm/llvm/bin"
TOOLS = ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf")

# (mangled name fragment, reason)
ALLOWED = [
    ("skinny_nh_kernel", "Li4ELi4ELi4ELb0E",
     "16-bit K x N decode, four activation tiles, no K split: 28 VGPRs spilled in the epilogue"),
]


def _kernels(so, tmp):
    fb = os.path.join(tmp, "fatbin.bin")
    subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fb}", so, os.path.join(tmp, "x.so")],
                   check=True, capture_output=True)
    data = open(fb, "rb").read()
    offs = [m.start() for m in re.finditer(b"__CLANG_OFFLOAD_BUNDLE__", data)] + [len(data)]
    out = []
    for i in range(len(offs) - 1):
        part, co = os.path.join(tmp, f"b{i}.bin"), os.path.join(tmp, f"b{i}.co")
        with open(part, "wb") as f:
            f.write(data[offs[i]:offs[i + 1]])
        subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={part}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"], check=True,
                       capture_output=True)
        notes = subprocess.run([f"{LLVM}/llvm-readelf", "--notes", co], check=True, capture_output=True,
                               text=True).stdout
        for blk in notes.split(".agpr_count:")[1:]:
            name = re.search(r"\.name:\s+(\S+)", blk).group(1)
            vs = int(re.search(r"\.vgpr_spill_count:\s+(\d+)", blk).group(1))
            ps = int(re.search(r"\.private_segment_fixed_size:\s+(\d+)", blk).group(1))
            out.append((name, vs, ps))
    return out


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    if not os.path.exists(ENGINE):
        pytest.skip("libvkblas_engine.so is not built")
    if not all(os.path.exists(os.path.join(LLVM, t)) for t in TOOLS):
        pytest.skip("the ROCm LLVM tools are missing")
    return _kernels(ENGINE, str(tmp_path_factory.mktemp("co")))


def test_every_kernel_family_is_present(kernels):
    names = " ".join(k[0] for k in kernels)
    for fam in ("gemm_pipe_kernel", "gemm_wavek_kernel", "gemm_kernel", "splitk_reduce_kernel", "gemv_kernel",
                "skinny_lds_kernel", "decode_lds_kernel", "skinny_n_kernel", "skinny_nh_kernel"):
        assert fam in names, fam


def test_no_kernel_spills_to_scratch(kernels):
    bad = []
    for name, vspill, scratch in kernels:
        if vspill == 0 and scratch == 0:
            continue
        if any(a in name and b in name for a, b, _ in ALLOWED):
            continue
        bad.append((name, vspill, scratch))
    assert not bad, bad


def test_allowed_spills_are_still_needed(kernels):
    """An allowance that no longer applies is removed from the list."""
    for a, b, why in ALLOWED:
        hits = [k for k in kernels if a in k[0] and b in k[0]]
        assert hits, (a, b)
        assert any(v or s for _, v, s in hits), why
