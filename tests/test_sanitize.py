"""The library's host code under AddressSanitizer + UndefinedBehaviorSanitizer
(CPU): tests/san/build.sh builds tests/san/san_driver.cpp against every
source with host-side instrumentation, and the driver reads a corpus of
damaged GGUF and llamafile images the way a loader does (GgufReader.open,
GgufReader.java:102-183; the ZIP / ZIP64 / forward-scan paths :808-1154).

Every file must fail cleanly -- JH_EFORMAT / JH_EIO (JH_EUNSUPPORTED for an
unknown tensor type) with a message -- or read consistently, and no sanitizer
may report.  The corpus: valid files of each kind, every truncation of the
header region, seeded byte corruptions, and hand-made hostile fields (counts
near 2^63, string and array lengths past the file, 9+ dimensions, dimension
products that overflow, data offsets past the end, bad alignment values, ZIP
directories and ZIP64 records pointing outside the file).
"""
import hashlib
import os
import struct
import subprocess

import numpy as np
import pytest

from gguf_build import (ARRAY, BOOL, FLOAT32, FLOAT64, INT8, INT32, STRING, UINT32, UINT64, _cd_entry, _eocd,
                        _local_header, _str, f32_bytes, gguf_bytes, llamafile, zip64_llamafile, STUB)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = os.path.join(ROOT, "tests", "san")
DRIVER = os.path.join(SAN, "_build", "san_driver")
STAMP = os.path.join(SAN, "_build", "stamp")


def _sources_hash():
    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "juno_amd", "csrc")
    files = [os.path.join(csrc, f) for f in sorted(os.listdir(csrc))]
    files += [os.path.join(ROOT, "include", "junohip.h"), os.path.join(SAN, "san_driver.cpp"),
              os.path.join(SAN, "build.sh")]
    for p in files:
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


@pytest.fixture(scope="module")
def driver():
    want = _sources_hash()
    if not (os.path.exists(DRIVER) and os.path.exists(STAMP) and open(STAMP).read() == want):
        r = subprocess.run(["bash", os.path.join(SAN, "build.sh")], capture_output=True, text=True, timeout=900)
        assert r.returncode == 0, r.stderr[-4000:]
        with open(STAMP, "w") as f:
            f.write(want)
    return DRIVER


def valid_gguf():
    meta = [("general.architecture", STRING, "llama"), ("general.alignment", UINT32, 32), ("k_bool", BOOL, True),
            ("k_str", STRING, "héllo"), ("k_arr", ARRAY, (INT32, [1, -2, 3])), ("k_f64", FLOAT64, 2.5),
            ("k_i8", INT8, -5), ("llama.context_length", UINT64, 4096),
            ("tokenizer.ggml.tokens", ARRAY, (STRING, ["a", "bb", "ccc"]))]
    rng = np.random.default_rng(0)
    q4 = rng.integers(0, 256, 144 * 2, dtype=np.uint8).tobytes()
    q8 = rng.integers(0, 256, 34 * 8, dtype=np.uint8).tobytes()
    tensors = [("t.f32", [4, 2], 0, f32_bytes(range(8))), ("t.q4k", [256, 2], 12, q4), ("t.q8", [32, 8], 8, q8)]
    return gguf_bytes(meta, tensors)


def header(n_tensors, n_kv, version=3):
    return struct.pack("<IiQQ", 0x46554747, version, n_tensors, n_kv)


def hostile_fields():
    """Hand-made headers with hostile counts, lengths, dims and offsets."""
    out = []
    big = [2 ** 63 - 1, 2 ** 62, 2 ** 40, 2 ** 32, 2 ** 31, 0xFFFFFFFF]
    for n in big:
        out.append(header(n, 0) + bytes(64))                           # tensor count
        out.append(header(0, n) + bytes(64))                           # metadata count
        out.append(header(0, 1) + struct.pack("<Q", n) + b"key")      # key length
        out.append(header(0, 1) + _str("k") + struct.pack("<iQ", STRING, n) + b"x")       # string value length
        out.append(header(0, 1) + _str("k") + struct.pack("<iiQ", ARRAY, INT32, n) + bytes(8))  # array count
        out.append(header(0, 1) + _str("k") + struct.pack("<iiQ", ARRAY, STRING, 2) + struct.pack("<Q", n))
        out.append(header(0, 1) + _str("k") + struct.pack("<iiQ", ARRAY, ARRAY, n) + bytes(16))  # nested arrays
        out.append(header(1, 0) + _str("t") + struct.pack("<i", 1) + struct.pack("<Q", n) + struct.pack("<iQ", 0, 0))
        out.append(header(1, 0) + _str("t") + struct.pack("<i", 2) + struct.pack("<QQ", n, n) + struct.pack("<iQ", 0, 0))
        out.append(header(1, 0) + _str("t") + struct.pack("<i", 1) + struct.pack("<Q", 4) + struct.pack("<iQ", 0, n))
        out.append(header(1, 0) + _str("t") + struct.pack("<i", 1) + struct.pack("<Q", 256) +
                   struct.pack("<iQ", 12, n))
    for nd in (-1, 0, 5, 8, 9, 255, 2 ** 31 - 1):
        out.append(header(1, 0) + _str("t") + struct.pack("<i", nd) + bytes(8 * 9) + struct.pack("<iQ", 0, 0))
    for t in (-1, 7, 9, 99, 2 ** 31 - 1):
        out.append(header(1, 0) + _str("t") + struct.pack("<i", 1) + struct.pack("<Q", 32) + struct.pack("<iQ", t, 0) +
                   bytes(64))
    for vt in (-1, 13, 99):
        out.append(header(0, 1) + _str("k") + struct.pack("<i", vt) + bytes(16))
    for a in (0, 1, 3, 2 ** 31, 2 ** 32 - 1):
        out.append(gguf_bytes([("general.alignment", UINT32, a)], [("t", [4], 0, f32_bytes([1, 2, 3, 4]))]))
    for v in (-1, 0, 1, 2, 4, 2 ** 31 - 1):
        out.append(header(0, 0, version=v))
    return out


def hostile_zips(g):
    out = []
    fn = b"m.gguf"
    body = bytearray(STUB) + _local_header(fn, len(g)) + g
    cd = _cd_entry(fn, len(g), len(STUB))
    ok = bytes(body + cd + _eocd(len(cd), len(body)))
    out.append(ok)
    n = len(ok)
    for cd_off in (n, n + 10, 2 ** 32 - 1, len(body) + 1, 0):
        out.append(bytes(body + cd + _eocd(len(cd), cd_off)))
    for cd_size in (0, 1, len(cd) + 1, 2 ** 32 - 1):
        out.append(bytes(body + cd + _eocd(cd_size, len(body))))
    for entries in (0, 2, 0xFFFF):
        out.append(bytes(body + cd + _eocd(len(cd), len(body), entries)))
    for lho in (len(body), n, 2 ** 32 - 2, len(STUB) + 1):
        c = _cd_entry(fn, len(g), lho)
        out.append(bytes(body + c + _eocd(len(c), len(body))))
    for size in (0, len(g) + 1, 2 ** 32 - 2):
        c = _cd_entry(fn, size, len(STUB))
        out.append(bytes(body + c + _eocd(len(c), len(body))))
    # name length past the directory
    c = bytearray(cd)
    struct.pack_into("<H", c, 28, 0xFFFF)
    out.append(bytes(body + c + _eocd(len(c), len(body))))
    # a local header whose name / extra lengths run past the file
    lh = bytearray(body)
    struct.pack_into("<HH", lh, len(STUB) + 26, 0xFFFF, 0xFFFF)
    out.append(bytes(lh + cd + _eocd(len(cd), len(body))))
    # ZIP64: records truncated or pointing outside
    z = bytearray(zip64_llamafile("m.gguf", g))
    out.append(bytes(z))
    loc_at = len(z) - 22 - 20
    for where in (2 ** 63 - 1, len(z), len(z) - 10, 0):
        zz = bytearray(z)
        struct.pack_into("<Q", zz, loc_at + 8, where)
        out.append(bytes(zz))
    for cut in range(1, 90, 7):
        out.append(bytes(z[: len(z) - cut]))
    # a ZIP with no entries at all, and a bare EOCD
    out.append(_eocd(0, 0, 0))
    out.append(STUB + _eocd(0, len(STUB), 0))
    return out


def corpus(tmp_path):
    g = valid_gguf()
    files = [g, llamafile("m.gguf", g), zip64_llamafile("m.gguf", g)]
    files += [g[:k] for k in range(0, min(len(g), 700))]
    files += [g[:k] for k in range(700, len(g), 29)]
    rng = np.random.default_rng(1234)
    for _ in range(600):
        b = bytearray(g)
        for _ in range(int(rng.integers(1, 5))):
            pos = int(rng.integers(0, min(len(b), 640)))
            b[pos] = int(rng.integers(0, 256))
        files.append(bytes(b))
    for _ in range(150):  # 8-byte fields overwritten with large values
        b = bytearray(g)
        pos = int(rng.integers(0, min(len(b), 600) - 8))
        struct.pack_into("<Q", b, pos, int(rng.choice([2 ** 63 - 1, 2 ** 62 + 7, 2 ** 32 + 1, 0xFFFFFFFF])))
        files.append(bytes(b))
    lf = llamafile("m.gguf", g)
    for _ in range(150):  # corruptions of the ZIP structures at the end of a llamafile
        b = bytearray(lf)
        for _ in range(int(rng.integers(1, 4))):
            pos = len(b) - 1 - int(rng.integers(0, 120))
            b[pos] = int(rng.integers(0, 256))
        files.append(bytes(b))
    files += hostile_fields() + hostile_zips(g)
    paths = []
    for i, data in enumerate(files):
        p = tmp_path / f"f{i:05d}.bin"
        p.write_bytes(data)
        paths.append(str(p))
    return paths


def test_reader_and_api_under_sanitizers(driver, tmp_path):
    paths = corpus(tmp_path)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([driver, *paths], capture_output=True, text=True, timeout=600, env=env)
    out = r.stdout + r.stderr
    print(out[-3000:])
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-6000:]
    assert r.returncode == 0, out[-6000:]
    assert f"san-driver files {len(paths)} unexpected 0" in r.stdout
