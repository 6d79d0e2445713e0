"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer.

* The CPU oracle (oracle/vs_oracle.cpp) driven through every entry point by
  oracle/sanitize_main.cpp on small seeded scenes: every camera model, the
  float, geometry, smooth-cutoff, brute-force, packed, Mip + floor, neural
  and surfel passes, both backwards, the camera gradient, the fused update,
  the SH step, the image loss, sort, scan and the codecs.
* The lagged-count capacity policy (vauss_amd/csrc/vs_capacity.h, the host
  side of the library's arena sizing) through tests/capacity_driver.cpp over
  window ends, growth, shrinking, many slots and the table's size limit.

Any out-of-bounds access, use after free, leak or undefined arithmetic
aborts the program (-fno-sanitize-recover=all), failing the test."""
import pathlib
import shutil
import subprocess

import pytest

REPO = pathlib.Path(__file__).resolve().parents[1]
SAN = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined,float-cast-overflow", "-fno-sanitize-recover=all",
       "-std=c++17"]


def _gxx():
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not available")
    return cxx


def test_oracle_under_asan_ubsan():
    _gxx()
    subprocess.run(["make", "-s", "-C", str(REPO / "oracle"), "sanitize"], check=True, capture_output=True)
    exe = REPO / "_build" / "sanitize" / "oracle_sanitize"
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600,
                         env={"ASAN_OPTIONS": "detect_leaks=1", "OMP_NUM_THREADS": "2", "PATH": "/usr/bin:/bin"})
    assert res.returncode == 0, res.stderr[-4000:]
    assert "oracle sanitizer run: ok" in res.stdout
    renders = int(res.stdout.split("(")[1].split()[0])
    assert renders >= 30


def test_capacity_policy_under_asan_ubsan(tmp_path):
    exe = tmp_path / "capacity_driver_san"
    subprocess.run([_gxx(), *SAN, "-o", str(exe), str(REPO / "tests" / "capacity_driver.cpp")], check=True)
    lines = []
    for slot in range(4):
        for r in range(450):                      # two full windows and a half per slot
            req = 200_000 + 3000 * ((r * 37 + slot * 11) % 97) + (4_000_000 if r == 300 else 0)
            lines.append(f"rec 1920 1080 {slot} {req} {100_000 + 10 * r} {1 << 31}")
            lines.append(f"hint 1920 1080 {slot} {150_000} {1 << 31}")
    for size in range(40):                        # past the table's limit of sizes: it is dropped
        lines.append(f"rec {64 + size} 64 0 {1000 + size} 500 {1 << 20}")
    lines += ["bucket 1e-12", "bucket 1e12", "bucket 0", "quantile 0.99 0.5 1 2 4 8 1e9 1e-9",
              "hint 1 1 200 1 1", "rec 1 1 0 0 0 1", "rec 1 1 0 4294967295 1 4294967295"]
    res = subprocess.run([str(exe)], input="\n".join(lines) + "\n", capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr[-4000:]
    out = res.stdout.strip().split("\n")
    assert len(out) == len(lines) and "error" not in out
