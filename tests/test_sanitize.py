"""AddressSanitizer + UndefinedBehaviorSanitizer runs of the CPU code that
reads untrusted or hand-built bytes, on the CPU (no GPU involved):

  * the loader's parsers (hawking_amd/csrc/hk_parse.cpp: HGRAV* containers,
    HQ30 payloads, GGUF Q4_0 blocks, the HQ80M15 catalog and its manifest),
    built with g++ into tests/sanitize/parse_harness.cpp and run on valid
    payloads from the same writer the GPU container tests use, on the
    rejection cases those tests check, and on every truncation and many
    single-byte mutations of each;
  * the oracle (oracle/hk_oracle.c, `make -C oracle sanitize`): the oracle's
    own test files run against the sanitized build in a subprocess.

Each run first shows that its sanitizers are live: a planted heap over-read
and signed overflow in the harness, and an undersized output buffer handed
to the sanitized oracle, must each stop the process with a report."""
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

from tests import hk_containers as W

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined", "-fno-sanitize-recover=all"]
ENV = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0", "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}

needs_gxx = pytest.mark.skipif(shutil.which("g++") is None or shutil.which("make") is None,
                               reason="needs g++ and make")


def _libasan():
    out = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    return os.path.realpath(out) if out and os.path.isabs(out) else None


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("san") / "parse_harness")
    cmd = ["g++", "-std=c++17", *SAN, "-Wall", "-Wextra", "-Werror", f"-I{ROOT}/include",
           f"-I{ROOT}/hawking_amd/csrc", f"{ROOT}/tests/sanitize/parse_harness.cpp",
           f"{ROOT}/hawking_amd/csrc/hk_parse.cpp", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def _run(exe, args):
    return subprocess.run([exe, *args], capture_output=True, text=True, env=dict(os.environ, **ENV), timeout=600)


@needs_gxx
def test_harness_sanitizers_are_live(harness):
    r = _run(harness, ["selftest-overread", "16"])
    assert r.returncode != 0 and "AddressSanitizer: heap-buffer-overflow" in r.stderr
    r = _run(harness, ["selftest-overflow", "5"])
    assert r.returncode != 0 and "signed integer overflow" in r.stderr


def _payloads(oracle, root):
    """(kind, path, should_accept) for valid payloads and rejection cases."""
    rows, cols = 4, 256
    s, g = oracle.bin_pack(oracle.deterministic_matrix(rows, cols, 19))
    p = oracle.rice_q1_pack(oracle.deterministic_matrix(8, 128, 23), 8, 128, 0.02)
    us, uc = oracle.uniform_pack(oracle.deterministic_matrix(3, 64, 29), 3, 64, 8, 64)
    L3 = oracle.uniform_pack(oracle.deterministic_matrix(64, 32, 3), 64, 32, 3, 64)
    R3 = oracle.uniform_pack(oracle.deterministic_matrix(32, 128, 5), 32, 128, 3, 64)
    hs, hc = oracle.q4_pack(oracle.deterministic_matrix(4, 128, 7), 64)
    bs8, bg8 = oracle.bin_pack(oracle.deterministic_matrix(8, 128, 9))
    q40 = np.random.default_rng(4).integers(0, 256, 2 * 64 // 32 * 18, dtype=np.uint8)
    q40[0::18] = 0x00
    q40[1::18] = 0x3C  # every block scale f16 1.0
    cases = [
        ("binary", W.binary(s, g, rows, cols), True),
        ("binary", W.binary(s, g, rows, cols, groups=int(s.size) + 1), False),
        ("binary", W.binary(s, g, rows, cols, shape=[rows, cols + 1]), False),
        ("binary", W.binary(s, g, rows, cols, elements=-1), False),
        ("binary", W.binary(s, g, rows, cols, groups=float(s.size)), False),
        ("binary", W.binary(s, g, rows, cols, shape=[2 ** 40, 2 ** 40]), False),
        ("residual", W.residual(p), True),
        ("residual", W.residual(p, index_bytes=5 + int(p.rice.size)), False),
        ("residual", W.residual(p, outlier_count=2 ** 62), False),
        ("residual", W.residual(p, rice_k=40), False),
        ("hgravs01", W.hgravs01(L3, R3, 64, 32, 128), True),
        ("hgravs01", W.hgravs01(L3, R3, 64, 32, 128, rank=16), False),
        ("hgravs01", W.hgravs01(L3, R3, 64, 32, 128, left_body_bytes=2 ** 63), False),
        ("uniform8", W.uniform8(us, uc, 3, 64), True),
        ("uniform8", W.uniform8(us, uc, 3, 64, group_size=32), False),
        ("hq30", W.hq30(b"HQ30UQ4\0", 64, [4, 128], hs, hc), True),
        ("hq30", W.hq30(b"HQ30G1B1", 128, [8, 128], bs8, bg8), True),
        ("hq30", W.hq30(b"HQ30UQ4\0", 64, [2, 2, 128], hs, hc), False),
        ("q4_0:2:64", q40.tobytes(), True),
        ("q4_0:2:64", q40.tobytes()[:-1], False),
    ]
    tensors = [("model.layers.0.mlp.experts.0.gate_proj.weight", 0, 1, [rows, cols], W.binary(s, g, rows, cols)),
               ("lm_head.weight", 3, 4, [3, 64], W.uniform8(us, uc, 3, 64))]
    mpath = W.write_catalog(root, tensors)
    cases.append(("catalog", (root / "catalog.hq80m15").read_bytes(), True))
    cases.append(("manifest", mpath.read_bytes(), True))
    out = []
    for i, (kind, payload, ok) in enumerate(cases):
        path = root / f"case_{i:02d}.bin"
        path.write_bytes(payload)
        out.append((kind, str(path), ok))
    return out


@needs_gxx
def test_parsers_under_asan_ubsan(oracle, harness, tmp_path):
    cases = _payloads(oracle, tmp_path)
    args = [a for kind, path, _ in cases for a in (kind, path)]
    r = _run(harness, args)
    assert r.returncode == 0, r.stderr[-4000:]
    lines = [l for l in r.stdout.splitlines() if " accepted=" in l]
    assert len(lines) == len(cases)
    for (kind, path, ok), line in zip(cases, lines):
        assert line.startswith(kind + " ") and f"accepted={int(ok)}" in line, (kind, path, line)
        assert int(line.split("variants=")[1]) > 100


@needs_gxx
def test_oracle_under_asan_ubsan():
    asan = _libasan()
    if not asan or not os.path.exists(asan):
        pytest.skip("libasan not found")
    r = subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "sanitize"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    env = dict(os.environ, **ENV, LD_PRELOAD=asan,
               HKO_ORACLE_LIB=os.path.join(ROOT, "oracle", "build", "asan", "libhk_oracle.so"))
    # live: an undersized output buffer (one float short) must stop the process
    planted = ("import numpy as np, ctypes as C\n"
               "from oracle import hk_oracle as o\n"
               "s, g = o.bin_pack(o.deterministic_matrix(8, 128, 3))\n"
               "out = np.empty(8 * 128 - 1, np.float32)\n"
               "o.lib().hko_bin_decode(o._ptr(s), o._ptr(g), 8, 128, 128, o._ptr(out))\n"
               "print('not stopped')\n")
    r = subprocess.run([sys.executable, "-c", planted], cwd=ROOT, env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode != 0 and "AddressSanitizer" in r.stderr, (r.stdout, r.stderr[-2000:])
    files = sorted(f for f in os.listdir(os.path.join(ROOT, "tests")) if f.startswith("test_oracle_"))
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                        *[os.path.join("tests", f) for f in files]],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert "passed" in r.stdout
