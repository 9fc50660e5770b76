"""The library's host code that reads untrusted input, under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU only; no GPU code is built).

The checkpoint parser (splatting-rs_amd/csrc/safetensors.cpp; the reference maps the same files,
depthanything3-rs/src/weights.rs:40-41, and the browser worker hands fetched bytes to
model_from_safetensors_bytes, weights.rs:51-60) and the host tables and size rules
(host_tables.cpp) are built with g++ together with tests/host/sanitize_main.cpp. Truncated files,
oversized lengths and integers, overflowing and negative shapes, bad escapes, runaway nesting and
wrong sizes must each come back as SPLAT_IO_ERROR (7) through both the mapped-file and the
byte-buffer loaders, and every run must finish without a sanitizer report.
"""
import json
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "splatting-rs_amd", "csrc")
IO_ERROR, BAD_ARGUMENT = 7, 1
SAN = ["-fsanitize=address,undefined,float-cast-overflow", "-fno-sanitize-recover=all"]


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    out = str(tmp_path_factory.mktemp("sanitize") / "sanitize_main")
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-ffp-contract=off", "-Wno-unknown-pragmas",
           *SAN, os.path.join(ROOT, "tests", "host", "sanitize_main.cpp"), os.path.join(CSRC, "safetensors.cpp"),
           os.path.join(CSRC, "host_tables.cpp"), "-o", out]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    return out


def _run(harness, *args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([harness, *args], capture_output=True, text=True, timeout=120, env=env)
    assert "runtime error" not in r.stderr and "Sanitizer" not in r.stderr, r.stderr[-3000:]
    assert r.returncode == 0, (r.returncode, r.stderr[-3000:])
    return r.stdout.splitlines()


def _file(header, data=b"", hlen=None):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    return struct.pack("<Q", len(h) if hlen is None else hlen) + h + data


def _valid():
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    b = np.array([0x3F80, 0xC000], np.uint16)          # bf16 1.0, -2.0
    c = np.array([0x3C00, 0x7BFF, 0x0001], np.uint16)  # f16 1.0, 65504, smallest subnormal
    data = a.tobytes() + b.tobytes() + c.tobytes()
    o1 = a.nbytes
    o2 = o1 + b.nbytes
    header = {"__metadata__": {"format": "pt", "x": [1.5, True, None, {"y": -2e-3}]},
              "a": {"dtype": "F32", "shape": [2, 3], "data_offsets": [0, o1]},
              "b\\u0041\"q": {"dtype": "BF16", "shape": [2], "data_offsets": [o1, o2]},
              "c": {"dtype": "F16", "shape": [3], "data_offsets": [o2, o2 + c.nbytes]}}
    h = json.dumps(header).replace("\\\\u0041", "\\u0041").encode()
    return _file(h, data)


def _malformed():
    v = _valid()
    t = lambda shape, offs, dtype="F32": {"t": {"dtype": dtype, "shape": shape, "data_offsets": offs}}
    return {
        "empty": b"",
        "short": b"\x01\x02\x03",
        "header past the end": _file(b"{}", hlen=1000),
        "header length 2^64-1": _file(b"{}", hlen=2 ** 64 - 1),
        "truncated header": _file(b'{"t": {"dtype": "F32", "sha'),
        "truncated data": v[:-3],
        "integer past int64": _file(b'{"t": {"dtype": "F32", "shape": [99999999999999999999], "data_offsets": [0, 4]}}', b"\0" * 4),
        "int64 min": _file(b'{"t": {"dtype": "F32", "shape": [-9223372036854775808], "data_offsets": [0, 4]}}', b"\0" * 4),
        "shape product overflow": _file(t([2 ** 32, 2 ** 32, 4], [0, 4]), b"\0" * 4),
        "byte size overflow": _file(t([2 ** 61, 2], [0, 4]), b"\0" * 4),
        "negative dimension": _file(t([-1, -4], [0, 16]), b"\0" * 16),
        "offsets past the data": _file(t([4], [0, 16]), b"\0" * 8),
        "reversed offsets": _file(t([0], [8, 0]), b"\0" * 8),
        "negative offset": _file(t([1], [-4, 0]), b"\0" * 8),
        "one offset": _file(t([1], [0]), b"\0" * 4),
        "size mismatch": _file(t([3], [0, 8]), b"\0" * 8),
        "unsupported dtype": _file(t([1], [0, 4], "X9"), b"\0" * 4),
        "bad \\u escape": _file(b'{"\\uZZZZ": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}', b"\0" * 4),
        "\\u at the end": _file(b'{"\\u12'),
        "nested metadata": _file(b'{"__metadata__": ' + b"[" * 100000 + b"]" * 100000 + b"}"),
        "unterminated string": _file(b'{"abc'),
        "garbage": _file(bytes(range(256)) * 4),
    }


def test_valid_checkpoint_parses_through_both_loaders(harness, tmp_path):
    path = tmp_path / "valid.safetensors"
    path.write_bytes(_valid())
    lines = _run(harness, "parse", str(path))
    # (0 + 1 + ... + 5) + (1 - 2) + (1 + 65504 + 2^-24), printed to 6 decimals
    assert lines == ["map OK 3 65519.000000", "bytes OK 3 65519.000000"], lines


@pytest.mark.parametrize("name", list(_malformed()))
def test_malformed_checkpoint_is_an_io_error(harness, tmp_path, name):
    path = tmp_path / "bad.safetensors"
    path.write_bytes(_malformed()[name])
    lines = _run(harness, "parse", str(path))
    assert len(lines) == 2, lines
    for line in lines:
        assert f" ERR {IO_ERROR} " in line, (name, line)


def test_host_tables_and_size_rules(harness):
    lines = _run(harness, "tables")
    res = {l.split(" OK ")[0] if " OK " in l else l.split(" ERR ")[0]: l for l in lines}
    errors = ["pos short", "rope -1", "uv 6 2x2", "uv 32 0x4", "da3_size 0x5", "da3_size -3x7",
              "ma_size 1x1073741824", "ma_size 1073741824x1", "ma_size 0x1", "ma_size none"]
    errors += [f"taps {f} 0->5" for f in (1, 2, 3, 4)] + [k for k in res if k.startswith("taps 4 ")]
    for k, line in res.items():
        want = " ERR " if k in errors else " OK "
        assert want in line, line
        if k.startswith("taps") and " OK " in line:
            assert float(line.split("sum_dev ")[1]) < 1e-5, line
    assert res["da3_size 4032x3024"].endswith("OK 504 378 504 378")
    assert res["ma_size 1000x700"].endswith("OK 518x392 cover 560x392")
    assert res["pos 1 37x37"].split(" OK ")[1].startswith("1370 ")
