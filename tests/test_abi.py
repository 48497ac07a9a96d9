"""CPU tests of the drop-in boundary: the C-ABI library loads, exports every
symbol include/*.h declares, and its host logic (argument checks, path
planning) behaves as documented.  No kernel is launched here."""
import ctypes
import importlib.util
import os
import re
import subprocess

import pytest

import vkblas_amd as vk

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(REPO, "include")


def declared_functions(header):
    text = open(os.path.join(INCLUDE, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w]*\s*\**\s+\**\s*([A-Za-z_]\w*)\s*\(", text, flags=re.M))
    # rocblas.h defines function-like macros of its GEMM names, so those
    # declarations parenthesise the name: rocblas_status(rocblas_gemm_ex)(...)
    names |= set(re.findall(r"^\s*[A-Za-z_]\w*\s*\(\s*(rocblas_\w+)\s*\)\s*\(", text, flags=re.M))
    names = {n for n in names if n.startswith(("vkblas_", "hipblas", "rocblas_"))}
    for decl, s, d, c, z in re.findall(r"^VKBLAS_FOUR\((\w+),\s*(\w+),\s*(\w+),\s*(\w+),\s*(\w+)\)", text, flags=re.M):
        for base in (s, d, c, z):
            names.add("hipblas" + base)
        names.add("hipblas" + c + "_v2")
        names.add("hipblas" + z + "_v2")
    return names


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", vk.LIB_PATH], check=True, capture_output=True, text=True)
    return {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}


def test_library_loads():
    L = vk.load()
    assert vk.version().startswith("vkblas-mi355x")
    assert L is vk.load()


@pytest.mark.parametrize("header", ["vkblas.h", "vkblas_ext.h", "vkblas_hipblas.h", "vkblas_rocblas.h",
                                    "vkblas_hipblaslt.h"])
def test_exports_every_declared_symbol(header):
    names = declared_functions(header)
    assert len(names) >= 3, names
    missing = sorted(names - exported_symbols())
    assert not missing, missing


def test_reference_export_set_present():
    """Symbols the reference's tests and PyTorch bind (test_gemm.c:212-215,
    test_h.c:84-86, test_v9h.c:51-52 and 144, src/vkblas_hipblas.c)."""
    want = {"hipblasSgemm", "hipblasCreate", "hipblasDestroy", "hipblasSgemmStridedBatched", "vkblas_gemm_bf16",
            "vkblas_gemm_f16", "vkblas_gemm_f32", "hipblasGemmEx", "hipblasGemmStridedBatchedEx_v2",
            "hipblasGemmEx_v2", "hipblasSetStream", "hipblasGetStream", "hipblasSetPointerMode",
            "hipblasGetPointerMode", "hipblasSetWorkspace", "vkblas_cache_invalidate_base",
            "hipblasHgemm", "hipblasHgemmStridedBatched", "hipblasGemmStridedBatchedEx",
            "rocblas_gemm_ex", "rocblas_gemm_strided_batched_ex"}
    assert not (want - exported_symbols())


def test_no_free_interposition():
    """The library must not export hipFree & co (no import cache to flush)."""
    assert not ({"hipFree", "hipHostFree", "hipFreeManaged"} & exported_symbols())


def _needed(path):
    out = subprocess.run(["readelf", "-d", path], check=True, capture_output=True, text=True).stdout
    return re.findall(r"\[(.*?)\]", "\n".join(l for l in out.splitlines() if "NEEDED" in l))


def test_no_cuda_or_oracle_dependency():
    """The drop-in library depends on no HIP runtime (LD_PRELOADed before an
    application's own runtime, it must not load one); the engine it opens
    depends on libamdhip64.so.7 and on nothing of CUDA, the oracle or the
    vendor BLAS libraries."""
    shim = _needed(vk.LIB_PATH)
    assert not any(n.startswith(("libamdhip64", "libhsa")) for n in shim), shim
    eng = _needed(vk.ENGINE_PATH)
    assert "libamdhip64.so.7" in eng, eng
    for needed in (shim, eng):
        assert not any("oracle" in n or "cuda" in n or "hipblas" in n or "rocblas" in n for n in needed), needed


def test_drop_in_references_no_hip_runtime_symbol():
    """Every HIP call goes through the engine: the drop-in's undefined symbols
    name no hip* runtime function (hipBLAS / hipBLASLt / rocBLAS ones are
    resolved at run time and not linked either)."""
    out = subprocess.run(["nm", "-D", "--undefined-only", vk.LIB_PATH], check=True, capture_output=True,
                         text=True).stdout
    undef = {line.split()[-1].split("@")[0] for line in out.splitlines() if line.strip()}
    assert not {u for u in undef if u.startswith(("hip", "rocblas", "hsa"))}, sorted(undef)


# --------------------------------------------------------------- planning

P = vk.plan


def test_hip_symbol_versions_within_torch_runtime():
    """Every versioned HIP symbol the library imports is defined by the HIP
    runtime PyTorch bundles: the library binds to that runtime inside a
    PyTorch process (same soname), and a newer symbol version would keep it
    from loading there."""
    import re
    import subprocess
    torch_rt = os.path.join(os.path.dirname(importlib.util.find_spec("torch").origin), "lib", "libamdhip64.so")
    if not os.path.exists(torch_rt):
        pytest.skip("no bundled HIP runtime in this torch")
    need = set(re.findall(r"\((hip_[0-9.]+)\)", subprocess.run(["objdump", "-T", vk.ENGINE_PATH], capture_output=True,
                                                               text=True, check=True).stdout))
    have = set(re.findall(r"\b(hip_[0-9.]+)\b", subprocess.run(["objdump", "-T", torch_rt], capture_output=True,
                                                               text=True, check=True).stdout))
    assert need and need <= have, sorted(need - have)


def test_plan_rejects_bad_arguments():
    with pytest.raises(vk.VkblasError):
        P(vk.DT_F32, vk.DT_F32, 0, 0, 0, 4, 4, 4, 4, 4)          # M == 0
    with pytest.raises(vk.VkblasError):
        P(vk.DT_F32, vk.DT_F32, 0, 0, 4, 4, 4, 4, 4, 4, batch=0)
    with pytest.raises(vk.VkblasError):
        P(vk.DT_F32, vk.DT_F32, 0, 0, 4, 4, 8, 0, 8, 4)          # lda == 0
    with pytest.raises(vk.VkblasError):
        P(vk.DT_F32, vk.DT_F32, 0, 0, 4, 8, 4, 4, 8, 0)          # ldc == 0
    # dimensions past the kernels' 32-bit signed indices: declined
    for M, N, K in ((1 << 31, 4, 4), (4, 1 << 31, 4), (4, 4, 1 << 31), (0xFFFFFFFF, 1, 1)):
        with pytest.raises(vk.VkblasError):
            P(vk.DT_F16, vk.DT_F16, 0, 0, M, N, K, K, N, N)
    assert P(vk.DT_F16, vk.DT_F16, 0, 0, (1 << 31) - 1, 1, 1, 1, 1, 1).path != vk.PATH_NONE
    # the engine contract takes leading dimensions as given (reference
    # test/test_h.c:105 passes lda = K + M%2 < M with op_a = T)
    assert P(vk.DT_F16, vk.DT_F16, 1, 0, 8, 4, 6, 6, 4, 4).path != vk.PATH_NONE
    with pytest.raises(vk.VkblasError):
        P(vk.DT_F16, vk.DT_BF16, 0, 0, 4, 4, 4, 4, 4, 4)         # f16 in, bf16 out: unsupported
    with pytest.raises(vk.VkblasError):
        P(vk.DT_BF16, vk.DT_F16, 0, 0, 4, 4, 4, 4, 4, 4)         # bf16 in, f16 out: unsupported
    # fp32 in, 16-bit out (GemmEx 32F/32F/16F and 16BF): a tile path (80
    # rows: more than the fp32 skinny kernels take)
    for ct in (vk.DT_F32, vk.DT_F16, vk.DT_BF16):
        assert P(vk.DT_F32, ct, 0, 0, 80, 4, 4, 4, 4, 4).path == vk.PATH_TILE64


def test_engine_param_errors_without_gpu():
    """Argument errors are reported before any device work (same codes as the
    reference: zero dims -> VKBLAS_ERR_PARAM, src/vkblas.c:3114)."""
    p = 4096
    assert vk.gemm_f32(0, 0, 0, 4, 4, 1.0, p, 4, p, 4, 0.0, p, 4) == vk.ERR_PARAM
    assert vk.gemm_f16(0, 0, 4, 4, 4, 1.0, None, 4, p, 4, 0.0, p, 4) == vk.ERR_PARAM
    assert vk.gemm_bf16(0, 0, 4, 0, 4, 1.0, p, 4, p, 4, 0.0, p, 4) == vk.ERR_PARAM
    # valid arguments with no GPU in the process: initialisation fails loudly
    assert vk.gemm_bf16(0, 0, 4, 4, 4, 1.0, p, 4, p, 4, 0.0, p, 4) == vk.ERR_INIT
    for name in ("vkblas_gemm_c64", "vkblas_gemm_f64", "vkblas_gemm_z64"):
        assert hasattr(vk.load(), name)


def test_plan_headline_configs():
    # config 2: fp32 4096^3 -> one 256x256 tile per CU
    for oa in (0, 1):
        for ob in (0, 1):
            pl = P(vk.DT_F32, vk.DT_F32, oa, ob, 4096, 4096, 4096, 4096, 4096, 4096)
            assert pl.path == vk.PATH_TILE256 and pl.split == 1
    # config 3: fp16 GEMMs
    for n in (2048, 4096, 8192):
        assert P(vk.DT_F16, vk.DT_F16, 0, 0, n, n, n, n, n, n).path in (vk.PATH_TILE128, vk.PATH_TILE256)
    # config 4: decode (engine op_a = N, op_b = T, M = tokens)
    for ntok in (1, 4, 8, 16, 17, 24):
        for dt in (vk.DT_F16, vk.DT_BF16):
            pl = P(dt, dt, 0, 1, ntok, 8192, 8192, 8192, 8192, 8192)
            assert pl.path == vk.PATH_SKINNY
    # up to 64 tokens at 8192^2: the decode kernels (weights above 12288 x
    # 4096 elements keep them for 33-64 rows too)
    for ntok in (32, 48, 64):
        assert P(vk.DT_F16, vk.DT_F16, 0, 1, ntok, 8192, 8192, 8192, 8192, 8192).path == vk.PATH_SKINNY
    # 65 tokens: a GEMM again
    assert P(vk.DT_F16, vk.DT_F16, 0, 1, 65, 8192, 8192, 8192, 8192, 8192).path != vk.PATH_SKINNY
    # not skinny when misaligned or batched
    assert P(vk.DT_F16, vk.DT_F16, 0, 1, 4, 8192, 8192, 8192, 8192, 8192, aligned=False).path != vk.PATH_SKINNY
    assert P(vk.DT_F16, vk.DT_F16, 0, 1, 4, 8192, 8192, 8192, 8192, 8192, batch=2).path != vk.PATH_SKINNY
    # config 5b: batched 64 x 512^3
    assert P(vk.DT_F32, vk.DT_F32, 0, 0, 512, 512, 512, 512, 512, 512, batch=64).split == 1


def test_plan_split_tail():
    """A partial last wave (at most half full) after whole waves of tiles:
    the last tile rows run split-K with as many slices as fit in one wave."""
    def pl(dt, M, N, K, **kw):
        return P(dt, dt, 0, 0, M, N, K, K, N, N, **kw)
    p = pl(vk.DT_F32, 3072, 3072, 3072)      # 24 x 24 tiles of 128: 512 + 64
    assert (p.path, p.tile, p.tail_rows, p.split, p.k_per_split) == (vk.PATH_TAIL, 1, 384, 7, 448)
    p = pl(vk.DT_F32, 5120, 5120, 5120)      # 40 x 40: 3 x 512 + 64
    assert (p.path, p.tail_rows, p.split) == (vk.PATH_TAIL, 256, 6)
    p = pl(vk.DT_F16, 6144, 6144, 6144)      # 24 x 24 tiles of 256: 2 x 256 + 64
    assert (p.path, p.tile, p.tail_rows, p.split) == (vk.PATH_TAIL, 2, 768, 3)
    p = pl(vk.DT_F32, 3000, 3072, 1024)      # ragged M: the tail holds the partial tile row
    assert (p.path, p.tail_rows) == (vk.PATH_TAIL, 3000 - 21 * 128)
    assert p.split * p.k_per_split >= 1024 > (p.split - 1) * p.k_per_split and p.k_per_split % 64 == 0
    # whole waves, a last wave more than half full, or under one wave: tiles only
    for dt, n in ((vk.DT_F32, 4096), (vk.DT_F32, 2048), (vk.DT_F16, 5120), (vk.DT_F16, 4096), (vk.DT_F32, 6144)):
        p = pl(dt, n, n, n)
        assert p.path in (vk.PATH_TILE128, vk.PATH_TILE256) and p.tail_rows == 0 and p.split == 1
    # a caller's split, never-split, batches and unaligned operands keep their plans
    assert pl(vk.DT_F32, 3072, 3072, 3072, split_k=1).path == vk.PATH_TILE128
    assert pl(vk.DT_F32, 3072, 3072, 3072, split_k=4).path == vk.PATH_SPLITK
    assert pl(vk.DT_F32, 3072, 3072, 3072, batch=2).path == vk.PATH_TILE128
    assert pl(vk.DT_F32, 3072, 3072, 3072, aligned=False).path != vk.PATH_TAIL


def test_plan_tile_crossover():
    """Square shapes where both pipelined tile sizes apply: fp32 keeps
    256x256 tiles only for about whole waves of one workgroup per CU; 16-bit
    inputs take them from 128 tiles on."""
    def tile(dt, n, batch=1):
        pl = P(dt, dt, 0, 0, n, n, n, n, n, n, batch=batch, split_k=1)   # no split tail
        assert pl.split == 1
        return pl.path
    T128, T256 = vk.PATH_TILE128, vk.PATH_TILE256
    assert [tile(vk.DT_F32, n) for n in (2048, 3072, 4096, 5120, 6144, 8192)] == [T128, T128, T256, T128, T128, T256]
    assert tile(vk.DT_F32, 512, batch=64) == T256          # 256 tiles: one whole wave
    assert tile(vk.DT_F32, 512, batch=60) == T256          # 240 of 256
    assert tile(vk.DT_F32, 512, batch=50) == T128          # 200 of 256
    for dt in (vk.DT_F16, vk.DT_BF16):
        assert [tile(dt, n) for n in (2048, 2560, 2816, 3072, 3584, 4096, 6144)] == [T128, T128, T128, T256, T256,
                                                                                      T256, T256]
    # exactly 128 tiles of 256x256 (half the CUs): 128x128 tiles; 144: 256x256
    for dt in (vk.DT_F16, vk.DT_BF16):
        for (m, n, k) in ((2048, 4096, 4096), (1024, 8192, 8192), (4096, 2048, 8192)):
            assert P(dt, dt, 0, 1, m, n, k, k, k, n, split_k=1).path == T128
        assert P(dt, dt, 0, 1, 4096, 2304, 4096, 4096, 4096, 2304, split_k=1).path == T256
        # and with a very long K, 2 slices of 256x256 tiles
        pl = P(dt, dt, 0, 1, 1024, 8192, 28672, 28672, 28672, 8192)
        assert (pl.path, pl.split, pl.tile) == (vk.PATH_SPLITK, 2, 2)
    # a shape only the generic kernels take keeps the size rule (fp32 5000^3: 256x256 tiles)
    assert P(vk.DT_F32, vk.DT_F32, 0, 0, 5000, 5000, 5000, 5000, 5000, 5000).path == T256


def test_plan_decode_split():
    """Decode K split: up to 16 tokens none; from 17 tokens the largest split
    that keeps the grid (128 weight rows per workgroup) within one round of
    256 workgroups, with at least 4 K steps of 128 per slice."""
    def split(M, N, K, ld=None):
        ld = ld or K
        pl = P(vk.DT_F16, vk.DT_F16, 0, 1, M, N, K, ld, ld, N)
        assert pl.path == vk.PATH_SKINNY
        return pl.split
    for M in (1, 2, 3, 16):
        assert split(M, 8192, 8192) == 1
    for M in (17, 24):
        assert split(M, 8192, 8192) == 4      # 64 workgroups per slice
        assert split(M, 14336, 4096) == 2     # 112 per slice: 224 workgroups
        assert split(M, 4096, 14336) == 8     # 32 per slice
    assert split(32, 4096, 14336) == 8
    # 33-64 rows: the decode kernels where the short-M tiles do not apply (K
    # below 4096, more than 128 column tiles, a weight above 12288 x 4096)
    assert split(64, 8192, 2048) == 4 and split(48, 40000, 8192) == 1
    assert split(64, 8192, 8192) == 4 and split(40, 14336, 4096) == 2 and split(64, 4096, 14336) == 8
    # and otherwise the short-M pipelined tiles with a K split
    for M, N, K in ((33, 4096, 8192), (64, 4096, 4096), (40, 11008, 4096), (64, 12288, 4096)):
        pl = P(vk.DT_F16, vk.DT_F16, 0, 1, M, N, K, K, K, N)
        assert (pl.path, pl.tile) == (vk.PATH_SPLITK, 1) and pl.split >= 2, (M, N, K)
    assert split(32, 256, 8192) == 16         # 2 per slice, 64 steps: 4 per slice
    assert split(32, 256, 1024) == 2          # 8 steps: at least 4 per slice
    assert split(32, 40000, 8192) == 1        # more than one round already
    assert split(20, 128, 100, ld=104) == 1   # a single (partial) K step


def test_plan_skinny_f32():
    """fp32 activation rows (op_a = N, fp32 output): the skinny kernels for up
    to 16 rows against W stored N x K (op_b = T, no split), the decode kernel
    for 17-64 rows against N x K, and K x N (op_b = N, M <= 16, N a
    multiple of 4, K split in whole 64-row groups so that the grid holds at
    most 256 workgroups of 128 columns, each slice at least 4 groups)."""
    for M in (1, 2, 4, 9, 16):
        for ob in (0, 1):
            pl = P(vk.DT_F32, vk.DT_F32, 0, ob, M, 8192, 8192, 8192, 8192, 8192)
            assert pl.path == vk.PATH_SKINNY
            assert pl.split == (1 if ob else 4)      # 64 column blocks x 4 slices
    assert P(vk.DT_F32, vk.DT_F32, 0, 0, 16, 4096, 14336, 14336, 4096, 4096).split == 8
    assert P(vk.DT_F32, vk.DT_F32, 0, 0, 1, 14336, 4096, 4096, 14336, 14336).split == 2
    assert P(vk.DT_F32, vk.DT_F32, 0, 0, 1, 1024, 65536, 65536, 1024, 1024).split == 32
    assert P(vk.DT_F32, vk.DT_F32, 0, 0, 3, 8192, 1000, 1000, 8192, 8192).split == 4
    assert P(vk.DT_F32, vk.DT_F32, 0, 0, 1, 4, 1, 4, 4, 4).split == 1
    # 17-64 rows against W stored N x K: the decode kernel, K split in
    # 64-float steps (8192^2: 64 workgroups of 128 rows x 4 slices)
    for M in (17, 40, 64):
        pl = P(vk.DT_F32, vk.DT_F32, 0, 1, M, 8192, 8192, 8192, 8192, 8192)
        assert pl.path == vk.PATH_SKINNY and pl.split == 4, (M, pl.path, pl.split)
    assert P(vk.DT_F32, vk.DT_F32, 0, 1, 65, 8192, 8192, 8192, 8192, 8192).path != vk.PATH_SKINNY
    # 17-64 rows against K x N: workgroups of 64 columns (8192^2: 128 of them
    # x 2 slices of 64 groups)
    for M in (17, 40, 64):
        pl = P(vk.DT_F32, vk.DT_F32, 0, 0, M, 8192, 8192, 8192, 8192, 8192)
        assert pl.path == vk.PATH_SKINNY and pl.split == 2, (M, pl.path, pl.split)
    assert P(vk.DT_F32, vk.DT_F32, 0, 0, 65, 8192, 8192, 8192, 8192, 8192).path != vk.PATH_SKINNY
    # not skinny: 16-bit output, N % 4 (K x N), op_a = T, misaligned leading
    # dimensions, ldb short of N
    assert P(vk.DT_F32, vk.DT_F16, 0, 1, 4, 8192, 8192, 8192, 8192, 8192).path != vk.PATH_SKINNY
    assert P(vk.DT_F32, vk.DT_F32, 0, 0, 4, 8190, 8192, 8192, 8192, 8192).path != vk.PATH_SKINNY
    assert P(vk.DT_F32, vk.DT_F32, 1, 1, 4, 8192, 8192, 8192, 8192, 8192).path != vk.PATH_SKINNY
    assert P(vk.DT_F32, vk.DT_F32, 0, 1, 4, 8192, 8190, 8190, 8192, 8192).path != vk.PATH_SKINNY
    assert P(vk.DT_F32, vk.DT_F32, 0, 0, 4, 8192, 8192, 8192, 8188, 8192).path != vk.PATH_SKINNY
    # one activation row: its leading dimension is never used
    assert P(vk.DT_F32, vk.DT_F32, 0, 1, 1, 8192, 8192, 3, 8192, 8192).path == vk.PATH_SKINNY
    # the staged N x K kernel's 32-bit buffer spans (32 weight rows of ldb)
    big = (1 << 31) // (32 * 4)
    assert P(vk.DT_F32, vk.DT_F32, 0, 1, 4, 4096, 4096, 4096, big - 4, 4096).path == vk.PATH_SKINNY
    assert P(vk.DT_F32, vk.DT_F32, 0, 1, 4, 4096, 4096, 4096, big, 4096).path != vk.PATH_SKINNY
    # the K x N kernel indexes with 64-bit offsets: no span limit
    assert P(vk.DT_F32, vk.DT_F32, 0, 0, 4, 4096, 4096, 4096, 1 << 30, 4096).path == vk.PATH_SKINNY


def test_plan_skinny_16bit_kn():
    """fp16 / bf16 with up to 64 activation rows and the weight stored K x N
    (op_b = N, PyTorch's x @ w): the 16-bit K x N kernel, N a multiple of 8,
    K split in 64-row groups so that the grid holds at most 256 workgroups of
    256 columns (M <= 16) or 128 columns (17 <= M <= 64), each slice at least
    4 groups."""
    for dt in (vk.DT_F16, vk.DT_BF16):
        for M in (1, 4, 16):
            pl = P(dt, dt, 0, 0, M, 8192, 8192, 8192, 8192, 8192)
            assert pl.path == vk.PATH_SKINNY and pl.split == 8     # 32 column blocks x 8 slices
        assert P(dt, vk.DT_F32, 0, 0, 3, 2048, 65536, 65536, 2048, 2048).split == 32
        assert P(dt, dt, 0, 0, 1, 14336, 4096, 4096, 14336, 14336).split == 4
        assert P(dt, dt, 0, 0, 16, 4096, 14336, 14336, 4096, 4096).split == 16
        assert P(dt, dt, 0, 0, 4, 8, 32, 32, 8, 8).split == 1
    for M in (17, 32, 64):
        assert P(vk.DT_F16, vk.DT_F16, 0, 0, M, 8192, 8192, 8192, 8192, 8192).split == 4   # 64 blocks x 4
    assert P(vk.DT_BF16, vk.DT_BF16, 0, 0, 64, 1000, 1032, 1032, 1000, 1000).split == 4
    # not this kernel: 65 rows, N % 8, ldb % 8, ldb short of N, lda % 8 (M > 1)
    assert P(vk.DT_F16, vk.DT_F16, 0, 0, 65, 8192, 8192, 8192, 8192, 8192).path != vk.PATH_SKINNY
    assert P(vk.DT_F16, vk.DT_F16, 0, 0, 4, 8188, 8192, 8192, 8192, 8188).path != vk.PATH_SKINNY
    assert P(vk.DT_F16, vk.DT_F16, 0, 0, 4, 8192, 8192, 8192, 8196, 8192).path != vk.PATH_SKINNY
    assert P(vk.DT_F16, vk.DT_F16, 0, 0, 4, 8192, 8192, 8192, 8184, 8192).path != vk.PATH_SKINNY
    assert P(vk.DT_F16, vk.DT_F16, 0, 0, 4, 8192, 8192, 8196, 8192, 8192).path != vk.PATH_SKINNY
    # one activation row: its leading dimension is never used
    assert P(vk.DT_BF16, vk.DT_BF16, 0, 0, 1, 8192, 8192, 3, 8192, 8192).path == vk.PATH_SKINNY


def test_plan_split_mid_size_m():
    """Mid-size M against a large weight (prefill-like shapes): at most 128
    output tiles of 128x128 and K >= 4096 split K so the grid fills the CUs.
    Pipelined 128x128 tiles (M >= 65 with K-major A; A rows past M read as
    row M - 1) take 256 / tiles slices; the generic kernel's tiles take
    min(K / 1024, 512 / tiles, 128)."""
    for dt in (vk.DT_F16, vk.DT_BF16, vk.DT_F32):
        for ob in (0, 1):
            def pl(M, N=8192, K=8192):
                return P(dt, dt, 0, ob, M, N, K, K, K if ob else N, N)
            assert (pl(128).path, pl(128).split, pl(128).tile) == (vk.PATH_SPLITK, 4, 1)     # 64 tiles
            assert (pl(256).path, pl(256).split) == (vk.PATH_SPLITK, 2)                      # 128 tiles
            assert (pl(192).path, pl(192).split) == (vk.PATH_SPLITK, 2)                      # 128 tiles, edge row
            assert (pl(65).path, pl(65).split, pl(65).tile) == (vk.PATH_SPLITK, 4, 1)        # short M, 64 tiles
            assert pl(384).split == 1 and pl(384).path != vk.PATH_SPLITK                     # 192 tiles
            assert pl(128, K=2048).split == 1                                                # K below 4096
    # fp32 from 17 to 64 rows: the decode kernels, W stored either way; short
    # M with MN-major A: the pipelined tiles with a K split
    assert P(vk.DT_F32, vk.DT_F32, 0, 0, 64, 4096, 4096, 4096, 4096, 4096).path == vk.PATH_SKINNY
    assert P(vk.DT_F32, vk.DT_F32, 0, 1, 64, 4096, 4096, 4096, 4096, 4096).path == vk.PATH_SKINNY
    pl = P(vk.DT_F16, vk.DT_F16, 1, 1, 96, 8192, 8192, 96, 8192, 8192)
    assert (pl.path, pl.split, pl.tile) == (vk.PATH_SPLITK, 8, 1)
    assert P(vk.DT_F16, vk.DT_F16, 0, 0, 1024, 1024, 8192, 8192, 1024, 1024).split == 4
    assert P(vk.DT_F16, vk.DT_F16, 0, 0, 2048, 1024, 8192, 8192, 1024, 1024).split == 2


def test_plan_decode_span_limit():
    """The decode kernels address a 32-row weight tile and the activation
    rows with 32-bit buffer offsets; a decode-shaped call whose leading
    dimensions exceed that span is planned on the tile path (which then
    runs), never as a skinny call the launcher would refuse."""
    big = (1 << 31) // (32 * 2)              # 32 rows of ldb fp16 elements reach 2 GiB
    assert P(vk.DT_F16, vk.DT_F16, 0, 1, 4, 4096, 4096, 4096, big - 8, 4096).path == vk.PATH_SKINNY
    assert P(vk.DT_F16, vk.DT_F16, 0, 1, 4, 4096, 4096, 4096, big, 4096).path != vk.PATH_SKINNY
    # activations: rows past M repeat row M - 1, so the span is (r - 1) lda
    # + K elements with r = M (M <= 16) or 16 ceil(M / 16) (counted as the
    # tiles the decode kernel stages, a bound on M)
    lim16 = ((1 << 30) - 4096) // 15 // 8 * 8   # largest lda with (15 lda + 4096) 2 bytes < 2 GiB
    assert P(vk.DT_F16, vk.DT_F16, 0, 1, 16, 4096, 4096, lim16, 4096, 4096).path == vk.PATH_SKINNY
    assert P(vk.DT_F16, vk.DT_F16, 0, 1, 16, 4096, 4096, lim16 + 8, 4096, 4096).path != vk.PATH_SKINNY
    lim32 = ((1 << 30) - 4096) // 31 // 8 * 8
    assert P(vk.DT_BF16, vk.DT_BF16, 0, 1, 17, 4096, 4096, lim32, 4096, 4096).path == vk.PATH_SKINNY
    assert P(vk.DT_BF16, vk.DT_BF16, 0, 1, 17, 4096, 4096, lim32 + 8, 4096, 4096).path != vk.PATH_SKINNY


@pytest.mark.parametrize("K", [65536, 262144])
@pytest.mark.parametrize("split", [4, 16, 64])
@pytest.mark.parametrize("dt", [vk.DT_F32, vk.DT_F16])
def test_plan_forced_split(K, split, dt):
    """config 5a: forced split factors; slices cover K exactly once, each
    slice a whole number of K steps and non-empty."""
    pl = P(dt, vk.DT_F32, 0, 0, 256, 256, K, K, 256, 256, split_k=split)
    assert pl.path == vk.PATH_SPLITK
    bk = 64 if dt == vk.DT_F16 else 32
    assert pl.k_per_split % bk == 0
    assert pl.split * pl.k_per_split >= K > (pl.split - 1) * pl.k_per_split
    assert pl.split == split
    # 64 slices of the four 128x128 tiles fill the CUs: the pipelined
    # 128x128 kernel; 16 slices of 64x64 tiles, or 4 slices of 64x64 tiles
    # each over four workgroups (tile code 4), do on the wave-K kernel
    assert pl.tile == {64: 1, 16: 0, 4: 4}[split]


def test_plan_split_heuristic_and_off():
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 256, 256, 65536, 65536, 256, 256)
    assert pl.path == vk.PATH_SPLITK and 2 <= pl.split <= 256
    # whole 128x128 tiles: pass 1 on the pipelined kernel, slices of whole
    # K-step pairs, about a workgroup per CU
    assert pl.tile == 1 and pl.k_per_split % 64 == 0 and 4 * pl.split <= 256
    # 16-bit inputs: the same
    pl = P(vk.DT_F16, vk.DT_F32, 0, 0, 256, 256, 262144, 262144, 256, 256)
    assert pl.path == vk.PATH_SPLITK and pl.tile == 1 and pl.k_per_split % 128 == 0 and 4 * pl.split <= 256
    # ragged M: 128x128 tiles (the pipelined pass 1 with a shifted edge tile),
    # slices of whole K-step pairs
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 200, 256, 65536, 65536, 256, 256)
    assert pl.path == vk.PATH_SPLITK and pl.tile == 1 and pl.k_per_split % 64 == 0 and 4 * pl.split <= 256
    # below the tile in M: from 65 rows (K-major A) the pipelined 128x128
    # pass 1 (rows past M read as row M - 1); up to 64 rows the decode kernel
    # (K-major A) or the generic 64x64 (MN-major A)
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 100, 256, 65536, 65536, 256, 256)
    assert pl.path == vk.PATH_SPLITK and pl.tile == 1 and pl.k_per_split % 64 == 0
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 60, 256, 65536, 65536, 256, 256)
    assert pl.path == vk.PATH_SKINNY and pl.split == 64
    pl = P(vk.DT_F32, vk.DT_F32, 1, 0, 60, 256, 65536, 60, 256, 256)
    assert pl.path == vk.PATH_SPLITK and pl.tile == 0
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 256, 256, 65536, 65536, 256, 256, split_k=1)
    assert pl.path != vk.PATH_SPLITK
    # batched calls never split
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 256, 256, 65536, 65536, 256, 256, batch=2, split_k=8)
    assert pl.split == 1
    # split count clamps so no slice is empty
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 64, 64, 100, 100, 64, 64, split_k=64)
    assert pl.split * pl.k_per_split >= 100 > (pl.split - 1) * pl.k_per_split


def test_preload_env_keeps_existing_preloads():
    """The preload list leads with this library and keeps what the
    environment already preloads; no HIP runtime is preloaded (the engine
    binds to the application's own)."""
    from vkblas_amd import preload, LIB_PATH
    env = preload.preload_env(base={"LD_PRELOAD": "/x/other.so"})
    assert env["LD_PRELOAD"].split(":") == [LIB_PATH, "/x/other.so"]
    assert preload.preload_env(base={})["LD_PRELOAD"] == LIB_PATH
    assert preload.main([]) == 2
    assert preload.torch_hipblas_command(["python3", "s.py", "-x"]) == ["python3", "-m", "vkblas_amd.torch_hipblas",
                                                                         "s.py", "-x"]
    # interpreter options stay with the interpreter
    assert preload.torch_hipblas_command(["python3", "-u", "-X", "dev", "s.py", "-u"]) == [
        "python3", "-u", "-X", "dev", "-m", "vkblas_amd.torch_hipblas", "s.py", "-u"]
    assert preload.torch_hipblas_command(["python3", "-u", "-m", "pkg.mod", "a"]) == [
        "python3", "-u", "-m", "vkblas_amd.torch_hipblas", "-m", "pkg.mod", "a"]
    for bad in (["python3"], ["python3", "-u"], ["python3", "-c", "print(1)"]):
        with pytest.raises(ValueError):
            preload.torch_hipblas_command(bad)


class _VkbEpi(ctypes.Structure):
    # vkb_epilogue_args (vkblas_amd/csrc/vkb_launch.h)
    _fields_ = [("c_in", ctypes.c_void_p), ("ldc_in", ctypes.c_int64), ("stride_c_in", ctypes.c_int64),
                ("bias", ctypes.c_void_p), ("bias_type", ctypes.c_int)]


class _VkbArgs(ctypes.Structure):
    # vkb_gemm_args (vkblas_amd/csrc/vkb_launch.h)
    _fields_ = [("A", ctypes.c_void_p), ("B", ctypes.c_void_p), ("C", ctypes.c_void_p),
                ("lda", ctypes.c_int64), ("ldb", ctypes.c_int64), ("ldc", ctypes.c_int64),
                ("stride_a", ctypes.c_int64), ("stride_b", ctypes.c_int64), ("stride_c", ctypes.c_int64),
                ("M", ctypes.c_uint32), ("N", ctypes.c_uint32), ("K", ctypes.c_uint32), ("batch", ctypes.c_uint32),
                ("split", ctypes.c_uint32), ("k_per_split", ctypes.c_uint32), ("stride_split", ctypes.c_int64),
                ("a_kmajor", ctypes.c_int), ("b_kmajor", ctypes.c_int), ("ab_type", ctypes.c_int),
                ("c_type", ctypes.c_int), ("alpha", ctypes.c_float), ("beta", ctypes.c_float),
                ("scalar_mode", ctypes.c_int), ("alpha_dev", ctypes.c_void_p), ("beta_dev", ctypes.c_void_p),
                ("generic_only", ctypes.c_int), ("ptr_array", ctypes.c_int),
                ("kernel_out", ctypes.POINTER(ctypes.c_int)), ("epi", ctypes.POINTER(_VkbEpi))]


@pytest.mark.parametrize("dt", [0, 1, 2])
def test_launcher_rejects_pointer_array_with_separate_c(dt):
    """The tile launcher refuses a pointer-array batch with a separate C
    input (no per-batch C_in pointers exist) and a pointer-array split, and
    decides it from the arguments alone: both return hipErrorInvalidValue (1)
    before any device call, so this runs without a GPU.  A regression test of
    the launcher reading its parameter block's pointer-array flag before
    setting it."""
    eng = ctypes.CDLL(vk.ENGINE_PATH)
    fn = eng.vkb_launch_gemm
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.POINTER(_VkbArgs), ctypes.c_int, ctypes.c_void_p]
    epi = _VkbEpi(c_in=0x10000, ldc_in=256, stride_c_in=0, bias=None, bias_type=0)
    a = _VkbArgs(A=0x1000, B=0x2000, C=0x3000, lda=256, ldb=256, ldc=256, M=256, N=256, K=256, batch=4,
                 split=1, k_per_split=256, a_kmajor=1, b_kmajor=1, ab_type=dt, c_type=dt, alpha=1.0, beta=1.0,
                 ptr_array=1, epi=ctypes.pointer(epi))
    for tile in (0, 1, 2):
        assert fn(ctypes.byref(a), tile, None) == 1
    a.epi = None
    a.split, a.k_per_split, a.stride_split = 2, 128, 65536
    assert fn(ctypes.byref(a), 1, None) == 1


def test_plan_caller_split_small_tiles():
    """A caller's split whose 128x128 tiles give fewer than 224 workgroups:
    split-K pass 1 on 64x64 tiles (the wave-K kernel) when they give at least
    224; else on 64x64 tiles with each K slice over four workgroups (tile code
    4) when that gives 224 and the slices are at least 16 K steps long; else
    on 32x32 tiles (tile code 3).  M = N = 256 at BASELINE configs[4]'s splits 4 / 16 / 64."""
    for dt in (vk.DT_F32, vk.DT_F16, vk.DT_BF16):
        for K in (65536, 262144):
            for split, tile in ((4, 4), (16, 0), (64, 1)):
                pl = P(dt, vk.DT_F32, 0, 0, 256, 256, K, K, 256, 256, split_k=split)
                assert (pl.path, pl.split, pl.tile) == (vk.PATH_SPLITK, split, tile), (dt, K, split, pl.tile)
    # ragged for 64x64 but whole 32x32 tiles: 32x32
    pl = P(vk.DT_F16, vk.DT_F32, 0, 0, 192, 96, 4096, 4096, 96, 96, split_k=5)
    assert (pl.path, pl.tile) == (vk.PATH_SPLITK, 3)
    # not whole 32x32 tiles: the generic kernel's 64x64 tiles
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 200, 96, 4096, 4096, 96, 96, split_k=5)
    assert (pl.path, pl.tile) == (vk.PATH_SPLITK, 0)
    # K not in whole 64-k steps: no wave-K plan for 16-bit inputs (fp32 steps are 32 k)
    pl = P(vk.DT_F16, vk.DT_F32, 0, 0, 256, 256, 8288, 8288, 256, 256, split_k=4)
    assert (pl.path, pl.tile) == (vk.PATH_SPLITK, 0)
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 256, 256, 8288, 8288, 256, 256, split_k=4)
    assert (pl.path, pl.tile) == (vk.PATH_SPLITK, 4)
    # slices too short to divide (fewer than 16 K steps of 32 k): 32x32
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 256, 256, 2048, 2048, 256, 256, split_k=4)
    assert (pl.path, pl.split, pl.tile) == (vk.PATH_SPLITK, 4, 4)
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 256, 256, 1024, 1024, 256, 256, split_k=4)
    assert (pl.path, pl.split, pl.tile) == (vk.PATH_SPLITK, 4, 3)
    # unaligned operands: no wave-K plan either
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 256, 256, 8192, 8192, 256, 256, split_k=4, aligned=False)
    assert (pl.path, pl.tile) == (vk.PATH_SPLITK, 0)


def test_plan_caller_split_collapsing_to_one_slice():
    """A split over a K within one slice runs a tile plan, never 32x32."""
    pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 256, 256, 32, 32, 256, 256, split_k=4)
    assert pl.split == 1 and pl.tile in (0, 1, 2)
    vk.set_override(-1, True)
    try:
        pl = P(vk.DT_F32, vk.DT_F32, 0, 0, 256, 256, 65536, 65536, 256, 256, split_k=4)
        assert (pl.path, pl.tile) == (vk.PATH_SPLITK, 0)
    finally:
        vk.set_override(-1, False)


_KNOB_SCRIPT = r"""
import sys
sys.path.insert(0, {repo!r})
import vkblas_amd as vk
P = vk.plan
out = []
for dt in (vk.DT_F32, vk.DT_F16):
    out.append(P(dt, vk.DT_F32, 0, 0, 4096, 4096, 4096, 4096, 4096, 4096).tile)
    out.append(P(dt, vk.DT_F32, 0, 0, 2048, 2048, 2048, 2048, 2048, 2048).tile)
    out.append(P(dt, vk.DT_F32, 0, 0, 256, 256, 65536, 65536, 256, 256).path)
    out.append(P(dt, vk.DT_F32, 0, 0, 256, 256, 65536, 65536, 256, 256, split_k=4).path)
print(out)
"""


@pytest.mark.parametrize("env,want", [
    ({}, [2, 1, 4, 4, 2, 1, 4, 4]),
    ({"VKBLAS_TILE128": "1"}, [1, 1, 4, 4, 1, 1, 4, 4]),
    ({"VKBLAS_TILE128": "0"}, [0, 0, 4, 4, 0, 0, 4, 4]),
    ({"VKBLAS_TILE128": "0", "VKBLAS_TILE": "256"}, [2, 2, 4, 4, 2, 2, 4, 4]),
    ({"VKBLAS_NOSPLITK": "1"}, [2, 1, 1, 4, 2, 1, 1, 4]),
    ({"VKBLAS_HSPLITK": "0"}, [2, 1, 4, 4, 2, 1, 1, 4]),
    ({"VKBLAS_HT256": "0"}, [2, 1, 4, 4, 1, 1, 4, 4]),
    ({"VKBLAS_HT256": "1"}, [2, 1, 4, 4, 2, 2, 4, 4]),
])
def test_reference_knob_names(env, want):
    """The reference's path knobs under their own names (src/vkblas.c:915,
    1356, 1637, 2858): per fp32 then fp16, the tile of 4096^3 and 2048^3,
    the path at M = N = 256, K = 65536 planned and with a caller's split 4
    (path 1 = 64x64 tiles, 4 = split-K).  Read once at load: one process
    per setting."""
    import json
    import sys
    e = dict(os.environ)
    for k in ("VKBLAS_TILE", "VKBLAS_TILE128", "VKBLAS_NOSPLITK", "VKBLAS_HSPLITK", "VKBLAS_HT256",
              "VKBLAS_SPLITK", "VKBLAS_KERNEL"):
        e.pop(k, None)
    e.update(env)
    r = subprocess.run([sys.executable, "-c", _KNOB_SCRIPT.format(repo=REPO)], env=e, capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert json.loads(r.stdout.strip().splitlines()[-1]) == want
