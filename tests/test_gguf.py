"""GGUF reader and weight pool (include/qlin_gguf.h) against files written by tests/gguf_writer.py.

The reference's parser (AI/codes/local-llm/src/format/gguf/GgufFile.cpp:152-247) has no tests of its
own and no .gguf fixture ships with it; these files are synthetic, written from the published format.
CPU tests cover parsing, metadata, tensor placement and every rejection; the GPU tests upload through
the pool and run kernels on the resident copies.
"""
import os
import struct

import numpy as np
import pytest

import gguf_writer as gw
import oracle as orc
import qgen
from blog_amd import gguf, qlin
from qgen import Q4_K, Q5_0, Q8_0, normwise_rel_err

OK, NULL, IO, FORMAT, NOT_FOUND = 0, 3, 8, 9, 10

META = [("general.architecture", gw.STRING, "qwen2"), ("qwen2.block_count", gw.U32, 28),
        ("qwen2.rope.freq_base", gw.F32, 1.0e6), ("general.file_type", gw.U32, 15),
        ("t.u8", gw.U8, 255), ("t.i8", gw.I8, -5), ("t.u16", gw.U16, 65535), ("t.i16", gw.I16, -300),
        ("t.i32", gw.I32, -7), ("t.u64", gw.U64, 2 ** 40 + 3), ("t.i64", gw.I64, -2 ** 40), ("t.f64", gw.F64, 0.125),
        ("t.bool", gw.BOOL, True), ("t.empty", gw.STRING, ""),
        ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, ["<s>", "hello", "", "world"])),
        ("tokenizer.ggml.token_type", gw.ARRAY, (gw.I32, [3, 1, 1, -2])),
        ("tokenizer.ggml.scores", gw.ARRAY, (gw.F32, [0.5, -1.25])),
        ("t.flags", gw.ARRAY, (gw.BOOL, [True, False, True]))]


def _tensors(seed=3):
    w4, rb4, _ = qgen.random_matrix(Q4_K, 32, 512, seed=seed)
    w8, rb8, _ = qgen.random_matrix(Q8_0, 7, 96, seed=seed + 1)
    w5, rb5, _ = qgen.random_matrix(Q5_0, 4 * 64, 128, seed=seed + 2)
    f = np.arange(5, dtype=np.float32)
    return [("blk.0.ffn_gate.weight", Q4_K, [32, 512], w4.tobytes()),
            ("blk.0.attn_k.weight", Q8_0, [7, 96], w8.tobytes()),
            ("output_norm.weight", 0, [5], f.tobytes()),
            ("blk.0.ffn_down_exps.weight", Q5_0, [4, 64, 128], w5.tobytes())]


@pytest.fixture
def written(tmp_path):
    path = tmp_path / "m.gguf"
    tensors = _tensors()
    start = gw.write(path, META, tensors)
    return path, tensors, start


def _status(path):
    h = __import__("ctypes").c_void_p()
    rc = qlin.lib().qlin_gguf_open(str(path).encode(), __import__("ctypes").byref(h))
    if rc == 0:
        qlin.lib().qlin_gguf_close(h)
    return rc


def test_header_tensors_and_placement(written):
    path, tensors, start = written
    with gguf.GgufFile(path) as f:
        assert f.version == 3 and f.alignment == 32
        assert f.tensor_view_names() == [t[0] for t in tensors]
        with open(path, "rb") as fh:
            raw = fh.read()
        for name, gtype, shape, data in tensors:
            v = f.get_tensor_view(name)
            assert v.dtype == gtype and list(v.shape) == shape          # file dims reversed: [out, in]
            assert v.nbytes == len(data) == gw.nbytes(gtype, shape)
            assert v.host_bytes() == data
            assert raw[start + v.offset:start + v.offset + v.nbytes] == data
        k = f.get_tensor_view("blk.0.ffn_gate.weight")
        assert k.row_bytes == qlin.row_bytes(Q4_K, 512) == 288
        assert f.get_tensor_view("blk.0.ffn_down_exps.weight").row_bytes == 64 * qlin.row_bytes(Q5_0, 128)
        assert not f.contain_tensor_view("missing.weight")
        with pytest.raises(qlin.QlinError):
            f.get_tensor_view("missing.weight")


def test_metadata_values(written):
    path, _, _ = written
    with gguf.GgufFile(path) as f:
        assert f.metadata_keys() == [k for k, _, _ in META]
        for key, vtype, value in META:
            got = f.metadata_value(key)
            if vtype == gw.ARRAY:
                et, items = value
                if et == gw.F32:
                    assert got == pytest.approx(items)
                elif et == gw.BOOL:
                    assert got == [int(b) for b in items]
                else:
                    assert got == items
            elif vtype == gw.F32:
                assert got == pytest.approx(value)
            else:
                assert got == value, key
        assert not f.contain_metadata("absent.key")
        L, h = qlin.lib(), f.handle
        import ctypes as C
        v = C.c_int64()
        assert L.qlin_gguf_get_i64(h, b"general.architecture", C.byref(v)) == NOT_FOUND   # a string
        assert L.qlin_gguf_get_i64(h, b"absent.key", C.byref(v)) == NOT_FOUND
        assert L.qlin_gguf_get_i64(h, b"t.u8", None) == NULL
        assert L.qlin_gguf_get_array_i64(h, b"tokenizer.ggml.token_type", 4, C.byref(v)) == NOT_FOUND
        info = qlin.GgufTensorInfo()
        assert L.qlin_gguf_tensor_info(h, 4, C.byref(info)) == NOT_FOUND
        assert L.qlin_gguf_find_tensor(h, b"nope") == -1


def test_alignment_and_version_2(tmp_path):
    """general.alignment moves the data section (GgufFile.cpp:192-198, 228-235); v2 files read alike."""
    tensors = _tensors(seed=11)
    for alignment, version in ((64, 3), (32, 2), (256, 3)):
        path = tmp_path / f"a{alignment}v{version}.gguf"
        meta = [("general.alignment", gw.U32, alignment)] if alignment != 32 else []
        start = gw.write(path, meta, tensors, version=version, alignment=alignment)
        assert start % alignment == 0
        with gguf.GgufFile(path) as f:
            assert f.alignment == alignment and f.version == version
            for name, _, _, data in tensors:
                assert f.get_tensor_view(name).host_bytes() == data
    # alignment 0 means the default 32
    path = tmp_path / "a0.gguf"
    gw.write(path, [("general.alignment", gw.U32, 0)], tensors)
    with gguf.GgufFile(path) as f:
        assert f.alignment == 32
        assert f.get_tensor_view(tensors[1][0]).host_bytes() == tensors[1][3]


def test_rejections(tmp_path):
    """Every case where the reference throws (GgufFile.cpp:152-247, 365-368) is a status here."""
    tensors = _tensors(seed=21)
    p = lambda n: tmp_path / f"{n}.gguf"  # noqa: E731
    assert _status(tmp_path / "does-not-exist.gguf") == IO
    gw.write(p("magic"), META, tensors, magic=b"GGUX")
    assert _status(p("magic")) == FORMAT
    gw.write(p("v1"), META, tensors, version=1)
    assert _status(p("v1")) == FORMAT
    gw.write(p("v4"), META, tensors, version=4)
    assert _status(p("v4")) == FORMAT
    gw.write(p("type"), META, tensors, type_override=99)           # unknown ggml type
    assert _status(p("type")) == FORMAT
    gw.write(p("partial"), META, tensors, dims_override=[300, 32])  # 9600 elements, not whole Q4_K blocks
    assert _status(p("partial")) == FORMAT
    gw.write(p("rows"), META, tensors, dims_override=[288, 64])    # whole blocks in all, not per row
    assert _status(p("rows")) == FORMAT
    gw.write(p("wrap"), META, tensors, dims_override=[1 << 40, 1 << 22], type_override=0)  # 2^64 bytes of F32
    assert _status(p("wrap")) == FORMAT
    gw.write(p("dims5"), META, tensors, dims_override=[512, 32, 1, 1, 1])
    assert _status(p("dims5")) == FORMAT
    gw.write(p("beyond"), META, tensors, offset_shift=1 << 20)      # data past the end of the file
    assert _status(p("beyond")) == FORMAT
    gw.write(p("full"), META, tensors)
    size = os.path.getsize(p("full"))
    for cut in (10, 23, 40, 200, size - 1):                       # truncated anywhere
        gw.write(p("cut"), META, tensors, truncate=cut)
        assert _status(p("cut")) == FORMAT, cut
    with open(p("badval"), "wb") as fh:                           # an unknown metadata value type
        fh.write(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 42)
                 + b"\0" * 16)
    assert _status(p("badval")) == FORMAT
    with open(p("hugecount"), "wb") as fh:                        # counts the file cannot hold
        fh.write(b"GGUF" + struct.pack("<IQQ", 3, 2 ** 40, 0) + b"\0" * 64)
    assert _status(p("hugecount")) == FORMAT
    assert qlin.lib().qlin_gguf_open(None, None) == NULL


# ---- device residency and kernels on the resident copies ------------------------------------

@pytest.mark.gpu
def test_pool_weights_drive_the_kernels(written):
    import torch
    from gpu_util import banner, bind_stream, empty_f32, host, dev
    path, tensors, _ = written
    banner("gguf pool weights")
    bind_stream()
    with gguf.GgufFile(path) as f, gguf.WeightPool() as pool:
        for name, qtype, k in (("blk.0.ffn_gate.weight", Q4_K, 512), ("blk.0.attn_k.weight", Q8_0, 96)):
            v = f.get_tensor_view(name)
            ptr, nb = pool.cached_weight(f, name)
            assert nb == v.nbytes and pool.cached_weight(f, name) == (ptr, nb)   # uploaded once
            n = v.shape[0]
            x = qgen.random_x(1, k, seed=k)
            y = empty_f32(n)
            qlin.call("qlin_launch_quant_gemv", qtype, ptr, v.row_bytes, dev(x), y, n, k, 1)
            w = np.frombuffer(v.host_bytes(), np.uint8)
            ref = orc.matmul_f64(qtype, w, v.row_bytes, x, n, k)
            assert normwise_rel_err(host(y), ref) <= 1e-5
        # expert views of the packed [4, 64, 128] Q5_0 tensor: expert e = base + e * nbytes / 4
        name = "blk.0.ffn_down_exps.weight"
        v = f.get_tensor_view(name)
        base, nb = pool.cached_weight(f, name)
        x = qgen.random_x(1, 128, seed=5)
        for e in range(4):
            ptr, eb, rows, cols = pool.expert_view(f, name, e)
            assert (eb, rows, cols) == (nb // 4, 64, 128) and ptr == base + e * eb
            y = empty_f32(rows)
            qlin.call("qlin_launch_quant_gemv", Q5_0, ptr, qlin.row_bytes(Q5_0, cols), dev(x), y, rows, cols, 1)
            w = np.frombuffer(v.host_bytes()[e * eb:(e + 1) * eb], np.uint8)
            ref = orc.matmul_f64(Q5_0, w, qlin.row_bytes(Q5_0, cols), x, rows, cols)
            assert normwise_rel_err(host(y), ref) <= 1e-5
        with pytest.raises(qlin.QlinError):
            pool.expert_view(f, name, 4)
        with pytest.raises(qlin.QlinError):
            pool.expert_view(f, "blk.0.ffn_gate.weight", 0)   # not a 3-D expert tensor
        assert pool.resident_bytes == sum(f.get_tensor_view(t[0]).nbytes for t in tensors if t[2] != [5])
        torch.cuda.synchronize()
