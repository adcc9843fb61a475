"""The libraries' host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

Both libraries are rebuilt with every host pass instrumented (`build.build_host_sanitized`: the
kernels' device code is unchanged), and `tests/sanitize/host_paths.cpp`, built with the same
clang's sanitizers, drives every host path a machine without a GPU reaches: the provider's entry
handshake, its JSON reader on 40,000 mutated OpKeys, repack of every served layout and its
refusals, the out-buffer protocol, per-thread messages; the C API's workspace sizing over
extreme shapes, the host repacks and argument refusals.  A sanitizer report aborts the run."""
import os
import shutil
import subprocess

import pytest

from syntropy_amd import build as B

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLANG = "/opt/rocm/llvm/bin/clang++"
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g"]
ENV = {"ASAN_OPTIONS": "detect_leaks=0", "UBSAN_OPTIONS": "print_stacktrace=1"}

pytestmark = pytest.mark.skipif(not (os.path.exists(B.HIPCC) and os.path.exists(CLANG)),
                                reason="needs hipcc and ROCm's clang++ with its sanitizer runtimes")


@pytest.fixture(scope="module")
def libs(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("sanitized"))
    hip, provider = B.build_host_sanitized(out)
    yield out, hip, provider
    shutil.rmtree(out, ignore_errors=True)


def _run(exe):
    env = dict(os.environ, **ENV)
    return subprocess.run([exe], capture_output=True, text=True, env=env, timeout=600)


def test_the_libraries_host_code_is_instrumented(libs):
    _, hip, provider = libs
    for lib in (hip, provider):
        undefined = subprocess.run(["nm", "-D", "--undefined-only", lib], capture_output=True, text=True,
                                   check=True).stdout
        assert "__asan_report_" in undefined and "__ubsan_handle_" in undefined, lib
    exported = subprocess.run(["nm", "-D", "--defined-only", provider], capture_output=True, text=True,
                              check=True).stdout.split()
    assert [s for s in exported if s.startswith("syntropy_")] == ["syntropy_provider_entry_v1@@SYNTROPY_PROVIDER_1"]


def test_the_runtime_reports_a_planted_overflow(tmp_path):
    """The harness itself: a heap overflow in a program built the same way is reported and fails."""
    src = tmp_path / "planted.cpp"
    src.write_text("#include <vector>\nint main(int c, char**) { std::vector<int> v(4); return v.data()[3 + c]; }\n")
    exe = str(tmp_path / "planted")
    subprocess.run([CLANG, *SAN, str(src), "-o", exe], check=True, capture_output=True)
    r = _run(exe)
    assert r.returncode != 0 and "heap-buffer-overflow" in r.stderr


def test_host_paths_run_clean_under_the_sanitizers(libs):
    out, _, _ = libs
    exe = os.path.join(out, "host_paths")
    subprocess.run([CLANG, "-std=c++17", "-O1", *SAN, os.path.join(ROOT, "tests", "sanitize", "host_paths.cpp"),
                    "-o", exe, f"-L{out}", "-l:libsyntropy_hip.so", "-l:libsyntropy_provider.so",
                    f"-Wl,-rpath,{out}", "-pthread"], check=True, capture_output=True)
    r = _run(exe)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-6000:]
    assert "all checks passed" in r.stdout
    assert "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-6000:]
