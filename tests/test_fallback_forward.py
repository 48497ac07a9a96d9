"""CPU tests of the engine-failure path of the drop-in library.

The reference forwards a GEMM to the real hipBLAS when its own engine fails
(src/vkblas_hipblas.c:244-246, 268-271) and forwards everything it does not
implement (src/vkblas_hipblas.c:467-532).  Here that path runs without a GPU:
the built libvkblas_hipblas.so is copied next to a fake libvkblas_engine.so
(tests/fake_layer/fake_engine.c, every GEMM returns a chosen status) and fake
vendor libraries with the real sonames (tests/fake_layer/fake_vendor.c,
libhipblas.so.3 and librocblas.so.5, each recording the call it receives).
Each case runs in a subprocess so the fakes never meet the real libraries.

Every case runs twice: against the built library, and against the drop-in
library rebuilt from its C / C++ sources with -fsanitize=address,undefined
(host code only: the drop-in library has no HIP code), with the ASan runtime
preloaded into the subprocess.
"""
import os
import shutil
import subprocess
import sys
import textwrap

import pytest

import vkblas_amd as vk

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE = os.path.join(REPO, "tests", "fake_layer")
CSRC = os.path.join(REPO, "vkblas_amd", "csrc")
ROCM = "/opt/rocm"


def _cc(out, srcs, extra=()):
    cmd = ["gcc", "-shared", "-fPIC", "-O1", "-std=gnu11", "-o", out, *srcs, "-I" + os.path.join(REPO, "include"),
           *extra]
    subprocess.run(cmd, check=True, capture_output=True, text=True)


def _sanitizer_runtime():
    out = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    return out if os.path.isabs(out) and os.path.exists(out) else None


@pytest.fixture(scope="module", params=["built", "sanitized"])
def layer(request, tmp_path_factory):
    d = tmp_path_factory.mktemp("fake_layer")
    if not os.path.exists(vk.LIB_PATH):
        pytest.fail(f"{vk.LIB_PATH} is not built")
    _cc(str(d / "libvkblas_engine.so"), [os.path.join(FAKE, "fake_engine.c")])
    _cc(str(d / "libhipblas.so.3"), [os.path.join(FAKE, "fake_vendor.c")], ["-DFAKE_HIPBLAS",
                                                                             "-Wl,-soname,libhipblas.so.3"])
    _cc(str(d / "librocblas.so.5"), [os.path.join(FAKE, "fake_vendor.c")], ["-DFAKE_ROCBLAS",
                                                                             "-Wl,-soname,librocblas.so.5"])
    env = dict(os.environ)
    if request.param == "sanitized":
        rt = _sanitizer_runtime()
        if rt is None:
            pytest.skip("no libasan for gcc")
        srcs = [os.path.join(CSRC, f) for f in ("engine_stub.c", "hipblas_shim.c", "rocblas_shim.c")]
        flags = ["-O1", "-g", "-fPIC", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
                 "-D__HIP_PLATFORM_AMD__", "-I" + ROCM + "/include", "-I" + CSRC, "-I" + os.path.join(REPO, "include")]
        objs = []
        for s in srcs:
            o = str(d / (os.path.basename(s) + ".o"))
            subprocess.run(["gcc", "-std=gnu11", "-c", s, "-o", o, *flags], check=True, capture_output=True, text=True)
            objs.append(o)
        o = str(d / "hipblaslt_shim.o")
        subprocess.run(["g++", "-std=c++17", "-c", os.path.join(CSRC, "hipblaslt_shim.cpp"), "-o", o, *flags],
                       check=True, capture_output=True, text=True)
        objs.append(o)
        subprocess.run(["g++", "-shared", "-fsanitize=address,undefined", "-o", str(d / "libvkblas_hipblas.so"),
                        *objs, "-ldl", "-lpthread"], check=True, capture_output=True, text=True)
        out = subprocess.run(["nm", "-D", str(d / "libvkblas_hipblas.so")], capture_output=True, text=True).stdout
        assert "__asan_init" in out and "__ubsan_handle" in out, "sanitizer instrumentation missing"
        env["LD_PRELOAD"] = rt
        env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
        env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    else:
        shutil.copy(vk.LIB_PATH, d / "libvkblas_hipblas.so")
    return str(d), env


PRELUDE = textwrap.dedent("""
    import ctypes, os, sys
    d = sys.argv[1]
    G = os.RTLD_GLOBAL | os.RTLD_NOW
    hb = ctypes.CDLL(os.path.join(d, "libhipblas.so.3"), mode=G)
    rb = ctypes.CDLL(os.path.join(d, "librocblas.so.5"), mode=G)
    L = ctypes.CDLL(os.path.join(d, "libvkblas_hipblas.so"))
    eng = ctypes.CDLL(os.path.join(d, "libvkblas_engine.so"))

    class Call(ctypes.Structure):
        _fields_ = [("fn", ctypes.c_char * 48), ("calls", ctypes.c_int), ("ta", ctypes.c_int), ("tb", ctypes.c_int),
                    ("m", ctypes.c_int64), ("n", ctypes.c_int64), ("k", ctypes.c_int64), ("lda", ctypes.c_int64),
                    ("ldb", ctypes.c_int64), ("ldc", ctypes.c_int64), ("batch", ctypes.c_int64),
                    ("A", ctypes.c_void_p), ("B", ctypes.c_void_p), ("C", ctypes.c_void_p),
                    ("alpha", ctypes.c_float), ("beta", ctypes.c_float)]
    for lib in (hb, rb):
        lib.fake_vendor_last.restype = ctypes.POINTER(Call)
    def last(lib):
        return lib.fake_vendor_last().contents
    def engine_mnk():
        a = (ctypes.c_uint32 * 3)()
        eng.fake_engine_last(a)
        return tuple(a)
    N, T = 111, 112
    A, B, C = ctypes.c_void_p(0x10000), ctypes.c_void_p(0x20000), ctypes.c_void_p(0x30000)
    alpha, beta = ctypes.c_float(1.5), ctypes.c_float(-0.25)
    h = ctypes.c_void_p()
    assert L.hipblasCreate(ctypes.byref(h)) == 0 and h.value
""")


def run_case(layer, body, status=None):
    d, env = layer
    env = dict(env)
    if status is not None:
        env["FAKE_ENGINE_STATUS"] = str(status)
    script = PRELUDE + textwrap.dedent(body) + "\nprint('CASE OK')\n"
    r = subprocess.run([sys.executable, "-c", script, d], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "CASE OK" in r.stdout, f"rc={r.returncode}\n{r.stdout}\n{r.stderr}"


def test_sgemm_engine_failure_forwards_unchanged(layer):
    """Engine error -> the vendor's hipblasSgemm gets the caller's arguments."""
    run_case(layer, """
        st = L.hipblasSgemm(h, N, T, 40, 24, 16, ctypes.byref(alpha), A, 40, B, 24, ctypes.byref(beta), C, 41)
        assert st == 0, st
        assert eng.fake_engine_calls() == 1
        assert engine_mnk() == (24, 40, 16), engine_mnk()   # column-major -> row-major swap
        c = last(hb)
        assert c.fn == b"hipblasSgemm" and c.calls == 1
        assert (c.ta, c.tb, c.m, c.n, c.k, c.lda, c.ldb, c.ldc) == (N, T, 40, 24, 16, 40, 24, 41)
        assert (c.A, c.B, c.C) == (A.value, B.value, C.value)
        assert (c.alpha, c.beta) == (1.5, -0.25)
    """)


def test_sgemm_engine_success_does_not_forward(layer):
    run_case(layer, """
        st = L.hipblasSgemm(h, N, N, 40, 24, 16, ctypes.byref(alpha), A, 40, B, 16, ctypes.byref(beta), C, 40)
        assert st == 0
        assert eng.fake_engine_calls() == 1
        assert last(hb).calls == 0
    """, status=0)


@pytest.mark.parametrize("status", [1, 2, 3])
def test_every_engine_error_forwards(layer, status):
    """VKBLAS_ERR_INIT / ERR_IMPORT / ERR_PARAM alike: the vendor computes."""
    run_case(layer, """
        st = L.hipblasSgemmStridedBatched(h, T, N, 8, 8, 8, ctypes.byref(alpha), A, 8, ctypes.c_longlong(64), B, 8,
                                          ctypes.c_longlong(64), ctypes.byref(beta), C, 8, ctypes.c_longlong(64), 3)
        assert st == 0
        assert eng.fake_engine_calls() == 1
        c = last(hb)
        assert c.fn == b"hipblasSgemmStridedBatched" and c.batch == 3 and (c.ta, c.tb) == (T, N)
    """, status=status)


def test_declined_shapes_never_reach_the_engine(layer):
    """m = 0 (quick return) and ld < rows (argument error) are the vendor's to
    report; the engine is not called."""
    run_case(layer, """
        assert L.hipblasSgemm(h, N, N, 0, 4, 4, ctypes.byref(alpha), A, 1, B, 4, ctypes.byref(beta), C, 1) == 0
        assert last(hb).fn == b"hipblasSgemm" and last(hb).m == 0
        assert L.hipblasSgemm(h, N, N, 8, 4, 4, ctypes.byref(alpha), A, 7, B, 4, ctypes.byref(beta), C, 8) == 0
        assert last(hb).lda == 7 and last(hb).calls == 2
        assert eng.fake_engine_calls() == 0
    """, status=0)


def test_gemm_ex_fp16_failure_forwards(layer):
    run_case(layer, """
        R16F, R32F, C32F = 2, 0, 2
        st = L.hipblasGemmEx(h, T, N, 64, 32, 128, ctypes.byref(alpha), A, R16F, 128, B, R16F, 128,
                             ctypes.byref(beta), C, R32F, 64, C32F, 0)
        assert st == 0, st
        assert eng.fake_engine_calls() == 1
        c = last(hb)
        assert c.fn == b"hipblasGemmEx" and (c.m, c.n, c.k) == (64, 32, 128)
    """)


def test_unimplemented_types_forward_without_engine(layer):
    """fp64 (hipblasDgemm) never touches the engine (reference forwarders,
    src/vkblas_hipblas.c:467-532)."""
    run_case(layer, """
        one = ctypes.c_double(1.0)
        st = L.hipblasDgemm(h, N, N, 4, 4, 4, ctypes.byref(one), A, 4, B, 4, ctypes.byref(one), C, 4)
        assert st == 0 and last(hb).fn == b"hipblasDgemm"
        assert eng.fake_engine_calls() == 0
    """, status=0)


def test_rocblas_engine_failure_forwards(layer):
    """The rocBLAS layer (PyTorch's fp16 path under hipBLAS) forwards too."""
    run_case(layer, """
        f16, f32 = 150, 151
        rh = ctypes.c_void_p()
        assert rb.rocblas_create_handle(ctypes.byref(rh)) == 0
        st = L.rocblas_gemm_ex(rh, T, N, 64, 32, 128, ctypes.byref(alpha), A, f16, 128, B, f16, 128,
                               ctypes.byref(beta), C, f16, 64, C, f16, 64, f32, 0, 0, 0)
        assert st == 0, st
        assert eng.fake_engine_calls() == 1
        c = last(rb)
        assert c.fn == b"rocblas_gemm_ex" and (c.m, c.n, c.k, c.ldc) == (64, 32, 128, 64)
        assert (c.alpha, c.beta) == (1.5, -0.25)
    """)


def test_partial_write_failure_is_reported_not_forwarded(layer):
    """VKBLAS_ERR_PARTIAL (5): a launch failed after a kernel writing part of
    C was enqueued (the split tail's head tiles).  Forwarding would let the
    vendor read those rows as its input C, so hipBLAS reports
    HIPBLAS_STATUS_EXECUTION_FAILED (5) and the vendor is not called."""
    run_case(layer, """
        st = L.hipblasSgemm(h, N, N, 40, 24, 16, ctypes.byref(alpha), A, 40, B, 16, ctypes.byref(beta), C, 40)
        assert st == 5, st
        assert eng.fake_engine_calls() == 1
        assert last(hb).calls == 0
    """, status=5)


def test_rocblas_partial_write_failure_is_reported_not_forwarded(layer):
    """The rocBLAS layer reports rocblas_status_internal_error (6) for it."""
    run_case(layer, """
        f16, f32 = 150, 151
        rh = ctypes.c_void_p()
        assert rb.rocblas_create_handle(ctypes.byref(rh)) == 0
        st = L.rocblas_gemm_ex(rh, T, N, 64, 32, 128, ctypes.byref(alpha), A, f16, 128, B, f16, 128,
                               ctypes.byref(beta), C, f16, 64, C, f16, 64, f32, 0, 0, 0)
        assert st == 6, st
        assert eng.fake_engine_calls() == 1
        assert last(rb).calls == 0
    """, status=5)
