"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer (the reference's
SIXI_ENABLE_SANITIZERS build, CMakeLists.txt:9,22-25): the C ABIs' validation and workspace
sizing (sixi_attn_abi.cpp, sixi_kv_abi.cpp, sixi_layer_abi.cpp, sixi_gdn_abi.cpp), the verify
planner (sixi_plan.cpp), the page pool (sixi_kv_pool.cpp) and the C oracle (fa_oracle.c),
driven by tests/sanitize/driver.cpp over random and edge-case descriptors, pool operation
sequences and small oracle cases.  Built on the host only (the device code of the ABI files
is compiled but never run); any sanitizer report fails the run."""
import os
import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
CSRC = ROOT / "sixi-asi_amd" / "csrc"
HOST_SOURCES = ["sixi_attn_abi.cpp", "sixi_kv_abi.cpp", "sixi_kv_pool.cpp", "sixi_plan.cpp", "sixi_layer_abi.cpp",
                "sixi_gdn_abi.cpp"]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and pathlib.Path(cand).exists():
            return cand
    return None


def _run(cmd, cwd):
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert proc.returncode == 0, " ".join(map(str, cmd)) + "\n" + proc.stdout[-4000:]
    return proc.stdout


def test_host_code_is_clean_under_asan_and_ubsan(tmp_path):
    hipcc = _hipcc()
    if hipcc is None or shutil.which("gcc") is None:
        pytest.skip("hipcc or gcc not available")
    inc = [f"-I{ROOT / 'include'}", f"-I{CSRC}", f"-I{ROOT / 'oracle'}"]
    # sanitizers on the host compilation only (each flag behind -Xarch_host)
    san_host = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]
    flags = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", *inc]
    objs = []
    for src in HOST_SOURCES + ["driver.cpp"]:
        path = CSRC / src if src != "driver.cpp" else ROOT / "tests" / "sanitize" / src
        obj = tmp_path / (src + ".o")
        _run([hipcc, *flags, *san_host, "-x", "hip", "-c", str(path), "-o", str(obj)], tmp_path)
        objs.append(obj)
    oracle_obj = tmp_path / "fa_oracle.o"
    _run(["gcc", "-O1", "-g", "-std=c11", "-fopenmp", "-ffp-contract=off", "-march=x86-64-v3", "-fsanitize=address",
          "-fsanitize=undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer",
          "-c", str(ROOT / "oracle" / "fa_oracle.c"), "-o", str(oracle_obj)], tmp_path)
    exe = tmp_path / "driver"
    _run([hipcc, "--offload-arch=gfx950", *san_host, "-fopenmp", "-o", str(exe), *map(str, objs), str(oracle_obj),
          "-lm"], tmp_path)
    # the OpenMP runtime's one-time thread-pool allocation is the only leak report; it is not ours
    supp = tmp_path / "lsan.supp"
    supp.write_text("leak:___kmp_allocate\n")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               LSAN_OPTIONS=f"suppressions={supp}", UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1",
               HIP_VISIBLE_DEVICES="", OMP_NUM_THREADS="2")
    proc = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, env=env,
                          timeout=300)
    out = proc.stdout
    assert proc.returncode == 0, out[-6000:]
    assert "sanitized host run: ok" in out, out[-3000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-6000:]
