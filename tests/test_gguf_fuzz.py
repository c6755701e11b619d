"""The GGUF reader (blog_amd/csrc/qlin_gguf.cpp) under the host sanitizers, over malformed files.

tests/gguf_fuzz_harness.cpp and the reader are compiled together with g++ and AddressSanitizer +
UndefinedBehaviorSanitizer (host code only: the reader has no device code), then run over the rejection
fixtures of test_gguf.py, every truncation of a valid file at 400 points, and seeded random mutations
of its header (bytes changed, extreme 4- and 8-byte counts and offsets written over fields, runs of
bytes deleted or inserted).  Every file must give QLIN_OK or a format/IO status, and no error path may
leak.  For an opened file the harness reads every byte the reader hands back, and checks each tensor's
data and each string against the file's own mapping in /proc/self/maps: a range inside it must end
within the file's size (the sanitizers do not see a read past the end of a file within its last page;
a harness built to read one byte past each tensor fails that check).  The reference
parser (AI/codes/local-llm/src/format/gguf/GgufFile.cpp:152-247) throws in the cases this one refuses.
"""
import os
import shutil
import struct
import subprocess
import sys

import numpy as np
import pytest

import gguf_writer as gw
from test_gguf import META, _tensors

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
N_MUTATIONS = 3000


def _write_cases(out):
    os.makedirs(out, exist_ok=True)
    p = lambda n: os.path.join(out, f"{n}.gguf")  # noqa: E731
    tensors = _tensors(seed=21)
    gw.write(p("valid"), META, tensors)
    gw.write(p("v2"), META, tensors, version=2)
    gw.write(p("align0"), [("general.alignment", gw.U32, 0)], tensors)
    gw.write(p("align64"), [("general.alignment", gw.U32, 64)], tensors)
    gw.write(p("magic"), META, tensors, magic=b"GGUX")
    gw.write(p("v1"), META, tensors, version=1)
    gw.write(p("v4"), META, tensors, version=4)
    gw.write(p("type"), META, tensors, type_override=99)
    gw.write(p("partial"), META, tensors, dims_override=[300, 32])
    gw.write(p("rows"), META, tensors, dims_override=[288, 64])
    gw.write(p("wrap"), META, tensors, dims_override=[1 << 40, 1 << 22], type_override=0)
    gw.write(p("dims5"), META, tensors, dims_override=[512, 32, 1, 1, 1])
    gw.write(p("beyond"), META, tensors, offset_shift=1 << 20)
    with open(p("badval"), "wb") as fh:
        fh.write(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 42)
                 + b"\0" * 16)
    with open(p("hugecount"), "wb") as fh:
        fh.write(b"GGUF" + struct.pack("<IQQ", 3, 2 ** 40, 0) + b"\0" * 64)
    with open(p("valid"), "rb") as fh:
        base = fh.read()
    for cut in range(0, len(base), max(1, len(base) // 400)):
        with open(p(f"cut{cut:06d}"), "wb") as fh:
            fh.write(base[:cut])
    # the metadata and the tensor table lie in the first ~1.2 KB; the data section follows
    hdr = min(len(base), 1200)
    rng = np.random.default_rng(20261202)
    extremes = [0, 1, 7, 13, 2 ** 31 - 1, 2 ** 31, 2 ** 32 - 1, 2 ** 32, 2 ** 40, 2 ** 63 - 1, 2 ** 63, 2 ** 64 - 1]
    for i in range(N_MUTATIONS):
        b = bytearray(base)
        kind = i % 4
        if kind == 0:
            for _ in range(int(rng.integers(1, 9))):
                b[int(rng.integers(0, hdr))] = int(rng.integers(0, 256))
        elif kind == 1:
            w = 8 if rng.integers(0, 2) else 4
            o = int(rng.integers(0, hdr - w))
            b[o:o + w] = (extremes[int(rng.integers(0, len(extremes)))] % (1 << (8 * w))).to_bytes(w, "little")
        elif kind == 2:
            o = int(rng.integers(0, hdr))
            del b[o:o + int(rng.integers(1, 64))]
        else:
            o = int(rng.integers(0, hdr))
            b[o:o] = bytes(rng.integers(0, 256, int(rng.integers(1, 64)), dtype=np.uint8))
        with open(p(f"mut{i:05d}"), "wb") as fh:
            fh.write(b)
    return sorted(os.path.join(out, f) for f in os.listdir(out))


@pytest.mark.skipif(shutil.which("g++") is None or not os.path.exists(os.path.join(ROCM, "include", "hip")),
                    reason="needs g++ and the HIP headers")
def test_reader_under_sanitizers(tmp_path):
    exe = str(tmp_path / "gguf_fuzz")
    # g++ only (the reader is host code); the HIP runtime is linked for the pool's calls, never reached here
    cmd = ["g++", "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-fno-omit-frame-pointer", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{ROOT}/include",
           os.path.join(ROOT, "tests", "gguf_fuzz_harness.cpp"), os.path.join(ROOT, "blog_amd", "csrc", "qlin_gguf.cpp"),
           f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    files = _write_cases(str(tmp_path / "cases"))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    opened = refused = 0
    for i in range(0, len(files), 500):  # argument lists of bounded length
        r = subprocess.run([exe, *files[i:i + 500]], capture_output=True, text=True, env=env, timeout=300)
        assert r.returncode == 0 and "ERROR" not in r.stderr and "runtime error" not in r.stderr, \
            (r.stdout[-2000:], r.stderr[-4000:])
        last = r.stdout.strip().splitlines()[-1].split()
        opened += int(last[1])
        refused += int(last[3])
    print(f"{len(files)} files: {opened} opened, {refused} refused", file=sys.stderr)
    assert opened + refused == len(files)
    assert opened >= 4 and refused >= 15  # the valid variants parse; every rejection fixture is refused
