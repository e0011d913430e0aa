"""AddressSanitizer + UndefinedBehaviorSanitizer run of the host code: the tape engine
(csrc/tape/*.cpp and the pybind11 module) and the C oracle, built with
-fsanitize=address,undefined in a scratch copy of the repository, then the CPU test suite
(`pytest -m "not gpu"`) run against those builds with gcc's ASan runtime preloaded.

Host only: GPU code is never built with a sanitizer (the kernel library, libgn_bwd.so, is
copied unsanitized; its host-side argument checks still run under the ASan runtime's
allocator).  Leak detection is off: the Python interpreter and torch keep allocations until
exit by design.  Any sanitizer report aborts the run (halt_on_error, no recovery).

Usage: python tests/sanitize_cpu.py [extra pytest args]      (not collected by pytest)
"""
import os
import shutil
import subprocess
import sys
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
       "-fno-omit-frame-pointer", "-g"]


def gcc_runtime(name):
    return subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True,
                          check=True).stdout.strip()


def scratch_copy(dst):
    ignore = shutil.ignore_patterns("_build", "__pycache__", "*.so", ".git", "gpurun_out", "_work",
                                    "profiles", ".pytest_cache")
    for d in ("tests", "oracle", "include", "grilly-next_amd"):
        shutil.copytree(os.path.join(ROOT, d), os.path.join(dst, d), ignore=ignore)
    # the kernel library is loaded as built (GPU code stays unsanitized)
    shutil.copy2(os.path.join(ROOT, "grilly-next_amd", "libgn_bwd.so"),
                 os.path.join(dst, "grilly-next_amd", "libgn_bwd.so"))


def main(argv):
    work = tempfile.mkdtemp(prefix="gn_sanitize_")
    try:
        scratch_copy(work)
        flags = " ".join(["-O1", "-fPIC", "-fopenmp", "-std=c11", "-Wall", "-Wno-unknown-pragmas",
                          "-D_GNU_SOURCE", *SAN])
        subprocess.run(["make", "-s", "-C", os.path.join(work, "oracle"), f"CFLAGS={flags}"],
                       check=True)
        pkg = os.path.join(work, "grilly-next_amd")
        subprocess.run([sys.executable, "-c",
                        "import sys; sys.path.insert(0, %r); import build_native as b; "
                        "print(b.build_tape(extra=%r))" % (pkg, SAN)], check=True)
        env = dict(os.environ)
        env["LD_PRELOAD"] = " ".join(p for p in (gcc_runtime("libasan.so"),
                                                 gcc_runtime("libubsan.so")) if os.path.isabs(p))
        env["ASAN_OPTIONS"] = ("detect_leaks=0:halt_on_error=1:abort_on_error=1:"
                               "alloc_dealloc_mismatch=0:new_delete_type_mismatch=0:"
                               "detect_odr_violation=0:protect_shadow_gap=0")
        env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
        cmd = [sys.executable, "-m", "pytest", os.path.join(work, "tests"), "-m", "not gpu", "-q",
               "-p", "no:cacheprovider", *argv]
        return subprocess.run(cmd, cwd=work, env=env).returncode
    finally:
        shutil.rmtree(work, ignore_errors=True)


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
