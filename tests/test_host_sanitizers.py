"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

* The C restatement of the oracle (``oracle/csrc/cl3_oracle.c``) is built with gcc's
  ASan + UBSan and the suite that calls it (``tests/test_oracle_ref_lib.py``: its
  tables, serial and OpenMP matmul and element-wise product on ragged and empty
  shapes) runs against it.
* The host side of the C-ABI library -- every ``.hip`` source, the device code built
  as usual -- is built with clang's ASan + UBSan, and ``tests/test_capi.py`` runs
  against it: every entry point's argument validation, size arithmetic and error
  reporting, none of which needs a GPU.

Each suite runs in a subprocess with its sanitizer runtime preloaded (the Python
interpreter is not instrumented).  Undefined behaviour aborts (-fno-sanitize-recover),
ASan aborts on its first error, and the output is searched for any report as well.
Leak checking is off: the interpreter keeps its allocations until exit.  The builds
go to ``*/_build/san`` (ignored by git) and are redone only when a source changed.
This file is not sent to the GPU box (``.gpurunignore``): nothing there builds.
"""

import glob
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
ORACLE_SRC = os.path.join(ROOT, "oracle", "csrc", "cl3_oracle.c")
ORACLE_SAN = os.path.join(ROOT, "oracle", "_build", "san", "libcl3_oracle.so")
HIP_DIR = os.path.join(ROOT, "yggdrasil_amd", "csrc")
HIP_SAN_DIR = os.path.join(ROOT, "yggdrasil_amd", "_build", "san")
HIP_SAN = os.path.join(HIP_SAN_DIR, "libygg_moe_san.so")
HIPCC = "/opt/rocm/bin/hipcc"
REPORTS = ("ERROR: AddressSanitizer", "runtime error:", "ERROR: LeakSanitizer", "SUMMARY: UndefinedBehavior")


def _stale(out, srcs):
    return not os.path.exists(out) or max(os.path.getmtime(s) for s in srcs) > os.path.getmtime(out)


def _run(cmd, **kw):
    res = subprocess.run(cmd, capture_output=True, text=True, **kw)
    assert res.returncode == 0, f"{' '.join(cmd[:3])} ... failed:\n{res.stdout[-3000:]}\n{res.stderr[-3000:]}"
    return res


def _build_oracle():
    if _stale(ORACLE_SAN, [ORACLE_SRC]):
        os.makedirs(os.path.dirname(ORACLE_SAN), exist_ok=True)
        _run(["gcc", "-std=c11", "-O1", "-g", "-fno-omit-frame-pointer", "-fPIC", "-ffp-contract=off", "-fopenmp",
              "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-shared", ORACLE_SRC, "-o",
              ORACLE_SAN])
    return ORACLE_SAN


def _build_hip():
    srcs = sorted(glob.glob(os.path.join(HIP_DIR, "*.hip")))
    deps = srcs + glob.glob(os.path.join(HIP_DIR, "*.h"))
    if _stale(HIP_SAN, deps):
        os.makedirs(HIP_SAN_DIR, exist_ok=True)
        # host-side instrumentation only: each sanitizer flag applies to the host pass
        host_san = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                    "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]
        flags = ["--offload-arch=gfx950", "-O2", "-g", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Xclang",
                 "-target-feature", "-Xclang", "-packed-fp32-ops", *host_san]
        procs = []
        objs = []
        for s in srcs:
            o = os.path.join(HIP_SAN_DIR, os.path.basename(s).replace(".hip", ".o"))
            objs.append(o)
            procs.append(subprocess.Popen([HIPCC, *flags, "-c", s, "-o", o], stdout=subprocess.PIPE,
                                          stderr=subprocess.PIPE, text=True))
        for p in procs:
            out, err = p.communicate()
            assert p.returncode == 0, err[-3000:]
        _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-shared-libsan", *host_san[:4], *objs, "-o",
              HIP_SAN])
    return HIP_SAN


def _clang_asan_runtime():
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


def _gcc_asan_runtime():
    path = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


def _pytest_under(preload, env_extra, files):
    env = dict(os.environ)
    env.update(env_extra)
    env["LD_PRELOAD"] = preload
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1:halt_on_error=1:detect_odr_violation=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m", "not gpu",
                          *files], cwd=ROOT, env=env, capture_output=True, text=True, timeout=1200)
    text = res.stdout + res.stderr
    for rep in REPORTS:
        assert rep not in text, text[-4000:]
    assert res.returncode == 0, text[-4000:]
    return text


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not found")
def test_oracle_c_restatement_under_asan_ubsan():
    rt = _gcc_asan_runtime()
    if rt is None:
        pytest.skip("gcc's ASan runtime not found")
    lib = _build_oracle()
    out = _pytest_under(rt, {"YGG_ORACLE_LIB": lib}, [os.path.join(ROOT, "tests", "test_oracle_ref_lib.py")])
    assert " passed" in out


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not found")
def test_c_abi_host_side_under_asan_ubsan():
    rt = _clang_asan_runtime()
    if rt is None:
        pytest.skip("clang's ASan runtime not found")
    lib = _build_hip()
    out = _pytest_under(rt, {"YGG_MOE_LIB": lib}, [os.path.join(ROOT, "tests", "test_capi.py")])
    assert " passed" in out
