"""GGUF checkpoints on the host: the Python writer and the library's native
parser (llmr_gguf_*) checked against each other and against the format's
fixed facts (header layout, ne order, 32-byte alignment), and every
truncation or corruption of a file rejected with an error, never a crash.
Host-only calls: no GPU needed."""
import os
import struct

import numpy as np
import pytest

from llmr_amd import capi, gguf
from llmr_amd import gguf_file as gf


@pytest.fixture(scope="module")
def lib():
    return capi.lib()


def _entries(r):
    w = (0.02 * r.standard_normal((64, 512))).astype(np.float32)
    v = r.standard_normal(96).astype(np.float32)
    return [gf.TensorEntry("blk.0.attn.weight", gguf.GGML_Q4_K, (64, 512), gf.encode_tensor(w, gguf.GGML_Q4_K)),
            gf.TensorEntry("blk.0.mlp.weight", gguf.GGML_Q8_0, (64, 512), gf.encode_tensor(w, gguf.GGML_Q8_0)),
            gf.TensorEntry("norm.scale", gguf.GGML_F32, (96,), gf.encode_tensor(v, gguf.GGML_F32)),
            gf.TensorEntry("emb.f16", gguf.GGML_F16, (3, 32), gf.encode_tensor(v[:96].reshape(3, 32), gguf.GGML_F16)),
            gf.TensorEntry("emb.bf16", gguf.GGML_BF16, (96,), gf.encode_tensor(v, gguf.GGML_BF16)),
            gf.TensorEntry("cube", gguf.GGML_F32, (2, 3, 4, 5), gf.encode_tensor(np.arange(120.0), gguf.GGML_F32))]


META = {"general.architecture": "flux", "u32": 7, "neg": -5, "big": 2 ** 40, "f": 0.5, "b": True,
        "ints": [1, 2, 3], "strs": ["a", "", "ccc"], "i8": gf.Typed(gf.T_INT8, -3),
        "u16": gf.Typed(gf.T_UINT16, 65535), "i16": gf.Typed(gf.T_INT16, -2), "u8": gf.Typed(gf.T_UINT8, 200),
        "f64": gf.Typed(gf.T_FLOAT64, 1e300), "f64s": gf.Typed(gf.T_ARRAY, (gf.T_FLOAT64, [1.5, -2.0])),
        "bools": gf.Typed(gf.T_ARRAY, (gf.T_BOOL, [True, False]))}


def test_round_trip_tensors_and_metadata(lib, tmp_path):
    r = np.random.default_rng(0)
    ents = _entries(r)
    p = str(tmp_path / "a.gguf")
    size = gf.write_gguf(p, ents, META)
    assert size == os.path.getsize(p)
    with gf.GGUFFile(p) as f:
        assert f.version == 3
        assert [t.name for t in f.tensors] == [e.name for e in ents]
        for t, e in zip(f.tensors, ents):
            assert t.ggml_type == e.ggml_type and t.shape == tuple(e.shape)
            assert t.ne == tuple(reversed(e.shape))           # ne fastest-varying first
            assert t.offset % 32 == 0                          # each tensor 32-aligned
            assert t.data_size == len(e.data)
            np.testing.assert_array_equal(f.host_bytes(t.name), np.frombuffer(e.data, np.uint8))
        md = f.metadata
    assert md["general.architecture"] == "flux" and md["u32"] == 7 and md["neg"] == -5 and md["big"] == 2 ** 40
    assert md["f"] == 0.5 and md["b"] is True and md["ints"] == [1, 2, 3] and md["strs"] == ["a", "", "ccc"]
    assert md["i8"] == -3 and md["u16"] == 65535 and md["i16"] == -2 and md["u8"] == 200 and md["f64"] == 1e300
    assert md["f64s"] == [1.5, -2.0] and md["bools"] == [True, False]


def test_header_and_alignment_facts(lib, tmp_path):
    """Header = <magic u32, version u32, n_tensors u64, n_kv u64>; tensor
    data starts at the first 32-byte boundary after the infos; offsets are
    relative to it (tools/gguf_writer.py:183-212, parser.c3:185-197)."""
    ents = _entries(np.random.default_rng(1))
    p = str(tmp_path / "b.gguf")
    gf.write_gguf(p, ents, {"k": 1})
    raw = open(p, "rb").read()
    assert raw[:24] == struct.pack("<IIQQ", 0x46554747, 3, len(ents), 1)
    with gf.GGUFFile(p) as f:
        last = f.tensors[-1]
    data_base = len(raw) - (last.offset + last.data_size + (-last.data_size) % 32)
    assert data_base % 32 == 0
    with gf.GGUFFile(p) as f:
        for t in f.tensors:
            assert raw[data_base + t.offset:data_base + t.offset + t.data_size] == ents[t.index].data


def _open_fails(lib, path):
    with pytest.raises(capi.LlmrError):
        gf.GGUFFile(path)


def test_every_truncation_is_an_error(lib, tmp_path):
    ents = [gf.TensorEntry("w", gguf.GGML_Q8_0, (2, 64), gf.encode_tensor(np.ones((2, 64)), gguf.GGML_Q8_0))]
    p = str(tmp_path / "c.gguf")
    gf.write_gguf(p, ents, {"name": "x", "arr": ["ab", "c"], "v": 3})
    raw = open(p, "rb").read()
    q = str(tmp_path / "t.gguf")
    pad = (-len(ents[0].data)) % 32  # cutting only the trailing padding leaves the tensor whole
    for n in range(len(raw) - pad):
        open(q, "wb").write(raw[:n])
        _open_fails(lib, q)
    open(q, "wb").write(raw[:len(raw) - pad])
    with gf.GGUFFile(q) as f:
        np.testing.assert_array_equal(f.host_bytes("w"), np.frombuffer(ents[0].data, np.uint8))


def test_corruptions_are_errors(lib, tmp_path):
    ents = [gf.TensorEntry("w", gguf.GGML_F32, (4,), gf.encode_tensor(np.ones(4), gguf.GGML_F32))]
    p = str(tmp_path / "d.gguf")
    gf.write_gguf(p, ents, {"v": 3})
    raw = bytearray(open(p, "rb").read())
    q = str(tmp_path / "e.gguf")

    def bad(mut):
        b = bytearray(raw)
        mut(b)
        open(q, "wb").write(bytes(b))
        _open_fails(lib, q)

    bad(lambda b: b.__setitem__(slice(0, 4), b"GGUG"))                       # magic
    bad(lambda b: b.__setitem__(slice(4, 8), struct.pack("<I", 4)))          # version 4
    bad(lambda b: b.__setitem__(slice(4, 8), struct.pack("<I", 1)))          # version 1
    bad(lambda b: b.__setitem__(slice(8, 16), struct.pack("<Q", 2 ** 60)))   # tensor count
    bad(lambda b: b.__setitem__(slice(16, 24), struct.pack("<Q", 2 ** 60)))  # key/value count
    # the key/value's type field (after its 8-byte length and 1-byte key "v")
    bad(lambda b: b.__setitem__(slice(33, 37), struct.pack("<I", 13)))       # unknown value type
    # the tensor info: name "w" then n_dims
    kv_end = 24 + 8 + 1 + 4 + 4
    bad(lambda b: b.__setitem__(slice(kv_end + 9, kv_end + 13), struct.pack("<I", 5)))  # 5 dims
    # 2^64 - 5 elements of Q4_K: ceil(n / 256) * 144 must not wrap to a size
    # that fits the file
    ne_pos = kv_end + 8 + 1 + 4

    def huge_q4k(b):
        b[ne_pos:ne_pos + 8] = struct.pack("<Q", 2 ** 64 - 5)
        b[ne_pos + 8:ne_pos + 12] = struct.pack("<I", gguf.GGML_Q4_K)
    bad(huge_q4k)
    # tensor offset past the file
    off_pos = kv_end + 8 + 1 + 4 + 8 + 4
    bad(lambda b: b.__setitem__(slice(off_pos, off_pos + 8), struct.pack("<Q", 1 << 20)))
    with pytest.raises(capi.LlmrError):
        gf.GGUFFile(str(tmp_path / "missing.gguf"))


def test_find_and_unknown_type_sizes(lib, tmp_path):
    import ctypes
    ents = [gf.TensorEntry("q", gguf.GGML_Q8_0, (1, 32), gf.encode_tensor(np.ones((1, 32)), gguf.GGML_Q8_0))]
    p = str(tmp_path / "f.gguf")
    gf.write_gguf(p, ents, {"a.key": 1})
    with gf.GGUFFile(p) as f:
        idx = ctypes.c_uint64()
        capi.check(lib.llmr_gguf_find_tensor(f._h, b"q", ctypes.byref(idx)))
        assert idx.value == 0
        assert lib.llmr_gguf_find_tensor(f._h, b"nope", ctypes.byref(idx)) == capi.LLMR_ERR_INVALID_ARG
        capi.check(lib.llmr_gguf_find_kv(f._h, b"a.key", ctypes.byref(idx)))
        assert lib.llmr_gguf_find_kv(f._h, b"b", ctypes.byref(idx)) == capi.LLMR_ERR_INVALID_ARG


def test_bf16_encoding_rounds_to_nearest_even_and_keeps_specials():
    """BF16 is the high half of the f32 pattern, rounded to nearest even;
    NaNs stay NaNs (a NaN whose payload sits in the low half would otherwise
    round to Inf, or carry into the sign), infinities and signed zeros stay
    as they are."""
    bits = np.array([0x3f800000, 0x3f808000, 0x3f818000, 0x3f808001, 0x7f7fffff,
                     0x7f800000, 0xff800000, 0x00000000, 0x80000000,
                     0x7f800001, 0xffffffff, 0x7fc00000, 0xff800001], np.uint32)
    out = np.frombuffer(gf.encode_tensor(bits.view(np.float32), gguf.GGML_BF16), "<u2")
    want = [0x3f80, 0x3f80, 0x3f82, 0x3f81, 0x7f80, 0x7f80, 0xff80, 0x0000, 0x8000]
    np.testing.assert_array_equal(out[:9], want)
    back = (out.astype(np.uint32) << 16).view(np.float32)
    assert np.isnan(back[9:]).all()
    assert (out[9:] & 0x0040).all()                            # quiet bit set
    np.testing.assert_array_equal(out[9:] >> 15, bits[9:] >> 31)  # sign kept
