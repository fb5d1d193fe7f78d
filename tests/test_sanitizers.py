"""AddressSanitizer and UndefinedBehaviorSanitizer over the host code, on the
CPU: the library's host side (ark_amd/csrc, `make asan`: every sanitizer flag
behind -Xarch_host, device code unchanged) and the oracle (oracle/, `make
asan`), both built by the ROCm clang so that one runtime -- clang's, preloaded
into a child Python -- serves the whole process.  Under it run the checkpoint
host parser's tests with their corruption fuzz, the ABI argument checks, and
the oracle's pin tests.  A planted heap overflow in a throwaway library built
the same way must be reported first, so a silent setup cannot pass."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.slow

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLANG = "/opt/rocm/llvm/bin/clang"
LIB = os.path.join(ROOT, "ark_amd", "lib", "asan", "libark_opt.so")
ORACLE = os.path.join(ROOT, "oracle", "_build", "asan", "libark_oracle.so")
TESTS = ["tests/test_ckpt_host_parse.py", "tests/test_abi.py", "tests/test_oracle_adam.py",
         "tests/test_oracle_amp.py", "tests/test_oracle_ckpt.py", "tests/test_oracle_clip.py",
         "tests/test_oracle_fp16.py", "tests/test_oracle_grad.py", "tests/test_oracle_norm.py",
         "tests/test_oracle_vector.py", "tests/test_golden.py", "tests/test_host_ckpt_order.py",
         "tests/test_oracle_grad_clip.py"]


def _runtime():
    if not os.path.exists(CLANG):
        pytest.skip("no ROCm clang")
    rt = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"],
                        stdout=subprocess.PIPE, text=True, check=True).stdout.strip()
    assert os.path.isabs(rt) and os.path.exists(rt), rt
    return rt


@pytest.fixture(scope="module")
def san_env():
    rt = _runtime()
    for d in ("oracle", os.path.join("ark_amd", "csrc")):
        r = subprocess.run(["make", "-C", os.path.join(ROOT, d), "asan"], stdout=subprocess.PIPE,
                           stderr=subprocess.STDOUT, text=True)
        assert r.returncode == 0, r.stdout[-3000:]
    env = dict(os.environ)
    env.update(LD_PRELOAD=rt, ARK_OPT_LIB=LIB, ARK_ORACLE_LIB=ORACLE,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    return env


def _run(env, args, cwd=ROOT):
    return subprocess.run([sys.executable] + args, cwd=cwd, env=env, stdout=subprocess.PIPE,
                          stderr=subprocess.STDOUT, text=True, timeout=900)


def test_a_planted_overflow_is_reported(san_env, tmp_path):
    src = tmp_path / "canary.c"
    src.write_text("#include <stdlib.h>\n"
                   "int canary(int i) { int *p = malloc(4 * sizeof(int)); p[0] = 1;\n"
                   "  int v = p[i]; free(p); return v; }\n")
    so = tmp_path / "libcanary.so"
    subprocess.run([CLANG, "-O1", "-g", "-fPIC", "-shared", "-fsanitize=address,undefined",
                    "-o", str(so), str(src)], check=True)
    code = f"import ctypes; L = ctypes.CDLL({str(so)!r}); print(L.canary(0)); print(L.canary(4))"
    r = _run(san_env, ["-c", code])
    assert r.returncode != 0 and "heap-buffer-overflow" in r.stdout, r.stdout[-2000:]


def test_sanitized_builds_are_the_ones_loaded(san_env):
    code = ("import oracle; from ark_amd._lib import lib; oracle.lib(); lib(); "
            "print(open('/proc/self/maps').read())")
    r = _run(san_env, ["-c", code])
    assert r.returncode == 0, r.stdout[-3000:]
    assert LIB in r.stdout and ORACLE in r.stdout and "libclang_rt.asan" in r.stdout


def test_host_parser_abi_checks_and_oracle_pins_run_clean(san_env):
    r = _run(san_env, ["-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu"] + TESTS)
    out = r.stdout
    assert r.returncode == 0, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert " passed" in out and " failed" not in out, out[-2000:]
