"""The library's host code under fault injection and the sanitizers (CPU
only; g++ builds from the library's own sources):
  - pool_fault_test.cpp against libqwmoe.so: every allocation inside every
    mutating slot-pool call made to throw in turn; each must return
    QWM_ERR_NOMEM and leave the pool as it was (the reference's
    throw-before-mutate contract, core/gpu_lru_pool_hooks.h:19-79, tested as
    tests/gpu_lru_index_test.cpp:12-22 does);
  - sanitize_driver.cpp with AddressSanitizer + UndefinedBehaviorSanitizer:
    signature-pool traces, and the GGUF index over valid, truncated and
    byte-corrupted files;
  - sanitize_driver.cpp with ThreadSanitizer: the file tier's reader
    threads."""
import os
import subprocess

import numpy as np
import pytest

from tests.gguf_file import GGML_F32, GGML_Q4_K, GGML_Q8_0, T_ARR, T_STR, T_U32, write_gguf
from tests.helpers import ROOT

CSRC = os.path.join(ROOT, "questwend_amd", "csrc")
HIP = ["-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include"]


def build(exe, sources, flags, libs=()):
    cmd = ["g++", "-std=c++17", "-g", "-O1", "-fno-omit-frame-pointer", "-pthread", *flags, "-o", exe, *sources, *libs]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]


def run(cmd, env_extra, timeout=600):
    env = dict(os.environ, **env_extra)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout, env=env)
    assert r.returncode == 0 and "runtime error" not in r.stderr and "Sanitizer" not in r.stderr, \
        (r.returncode, r.stdout[-2000:], r.stderr[-6000:])
    return r.stdout


def test_pool_throws_before_mutating(tmp_path):
    lib = os.path.join(ROOT, "questwend_amd")
    exe = str(tmp_path / "pool_fault")
    build(exe, [os.path.join(ROOT, "tests", "pool_fault_test.cpp")], ["-Wno-mismatched-new-delete"],
          ["-L" + lib, "-lqwmoe", "-Wl,-rpath," + lib])
    out = run([exe, str(tmp_path)], {})
    assert out.startswith("ok ") and int(out.split()[1]) >= 100, out


def gguf_files(tmp_path):
    """A valid file, then every 97th truncation of it and 150 copies with
    random bytes overwritten in the header and tensor index."""
    rng = np.random.default_rng(5)
    ts = [("token_embd.weight", GGML_Q8_0, [512, 4], rng.integers(0, 256, 4 * 16 * 34, dtype=np.uint8).tobytes()),
          ("output_norm.weight", GGML_F32, [512], rng.integers(0, 256, 2048, dtype=np.uint8).tobytes())]
    for b in range(2):
        for role in ("gate", "up", "down"):
            ne = [512, 256, 4] if role != "down" else [256, 512, 4]
            ts.append((f"blk.{b}.ffn_{role}_exps.weight", GGML_Q4_K, ne,
                       rng.integers(0, 256, 4 * 73728, dtype=np.uint8).tobytes()))
    kvs = [("general.architecture", T_STR, "qwen3moe"), ("a.arr", T_ARR, (T_STR, ["x", "yz"])),
           ("a.n", T_U32, 3)]
    good = tmp_path / "good.gguf"
    write_gguf(str(good), kvs, ts, alignment=64)
    blob = good.read_bytes()
    head = 2048
    files = [str(good)]
    for cut in range(0, min(len(blob), 8192), 97):
        f = tmp_path / f"cut{cut}.gguf"
        f.write_bytes(blob[:cut])
        files.append(str(f))
    for i in range(150):
        b = bytearray(blob[:head + 4096])
        for _ in range(int(rng.integers(1, 6))):
            b[int(rng.integers(0, head))] = int(rng.integers(0, 256))
        f = tmp_path / f"flip{i}.gguf"
        f.write_bytes(bytes(b))
        files.append(str(f))
    return files


def test_pool_and_gguf_under_asan_ubsan(tmp_path):
    exe = str(tmp_path / "san")
    build(exe, [os.path.join(ROOT, "tests", "sanitize_driver.cpp"), os.path.join(CSRC, "qwm_pool.cpp"),
                os.path.join(CSRC, "qwm_gguf.cpp"), os.path.join(CSRC, "qwm_error.cpp")],
          ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", *HIP],
          ["-L/opt/rocm/lib", "-lamdhip64"])
    supp = tmp_path / "lsan.supp"
    supp.write_text("leak:libamdhip64\nleak:libhsa-runtime64\nleak:librocprofiler\n")
    env = {"ASAN_OPTIONS": "halt_on_error=1:detect_leaks=1", "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1",
           "LSAN_OPTIONS": f"suppressions={supp}"}
    run([exe, "pool", str(tmp_path)], env)
    out = run([exe, "gguf", *gguf_files(tmp_path)], env)
    assert int(out.split()[-1]) >= 4, out      # the valid file's lookups succeed


def test_reader_threads_under_tsan(tmp_path):
    exe = str(tmp_path / "tsan")
    build(exe, [os.path.join(ROOT, "tests", "sanitize_driver.cpp")],
          ["-fsanitize=thread", "-DQWM_SAN_READERS_ONLY"])
    out = run([exe, "readers"], {"TSAN_OPTIONS": "halt_on_error=1"})
    assert "readers ok" in out
