"""The GGUF reader (laplace_amd.gguf, following GGUFContext::open,
src/gguf.cpp:209-389) on files written by the reference's own test writer
(tests/gguf_writer.h, compiled unmodified into oracle/_ref): every metadata
value kind the writer emits, tensors of several types and ranks with
unaligned sizes, the 32-byte data alignment, and truncation. Offsets and
the data-section start are computed here from the format (header, then
tensor infos, padded to 32; tensors packed at 32-byte multiples), and the
bytes the reader returns are compared exactly with the bytes handed to the
writer."""
import numpy as np
import pytest

from laplace_amd.gguf import GGUFError, GGUFFile, tensor_nbytes

F32, F16, Q4_0, Q8_0, Q2_K, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 10, 12, 13, 14


@pytest.fixture()
def writer(ref, orc):
    return orc.RefGGUFWriter


def _tensors(rng):
    spec = [("token_embd.weight", Q8_0, (64, 3)), ("blk.0.attn_q.weight", Q4_K, (512, 5)),
            ("blk.0.ffn_down.weight", Q6_K, (256, 3)), ("blk.0.ffn_up.weight", Q5_K, (256, 2, 2)),
            ("blk.0.ffn_gate.weight", Q2_K, (256, 1)), ("blk.0.attn_k.weight", Q4_0, (96, 2)),
            ("output_norm.weight", F32, (33,)), ("rope_freqs", F16, (7,))]
    out = []
    for name, t, dims in spec:
        nb = tensor_nbytes(t, dims)
        out.append((name, t, dims, rng.integers(0, 256, nb, dtype=np.uint8)))
    return out


def _write(writer, path, tensors, meta, truncate=0):
    w = writer()
    for kind, key, value in meta:
        w.kv(kind, key, value)
    for name, t, dims, data in tensors:
        w.tensor(name, dims, t, data)
    w.write(path, truncate)


def _header_bytes(tensors, meta):
    """Bytes before the data section, from the GGUF v3 layout: magic,
    version, two u64 counts; each KV = key (u64 len + bytes), u32 type,
    value; each tensor info = name, u32 ndims, u64 dims, u32 type, u64
    offset."""
    s = lambda v: 8 + len(v.encode())
    n = 4 + 4 + 8 + 8
    for kind, key, value in meta:
        n += s(key) + 4
        n += {"u32": 4, "i32": 4, "f32": 4, "bool": 1}.get(kind, 0)
        if kind == "str":
            n += s(value)
        elif kind.startswith("arr_"):
            n += 4 + 8
            if kind == "arr_str":
                n += sum(s(v) for v in value)
            else:
                n += len(value) * {"arr_u8": 1, "arr_i16": 2, "arr_bool": 1, "arr_i32": 4}[kind]
    for name, t, dims, data in tensors:
        n += s(name) + 4 + 8 * len(dims) + 4 + 8
    return n


META = [("u32", "gemma4.block_count", 30), ("i32", "neg", -7), ("f32", "gemma4.rope.freq_base", 1.0e6),
        ("bool", "flag", True), ("bool", "off", False), ("str", "general.architecture", "gemma4"),
        ("arr_str", "tokenizer.ggml.tokens", ["<s>", "a", "bc", ""]), ("arr_u8", "bytes", [0, 7, 255]),
        ("arr_i16", "shorts", [-2, 3, 32767]), ("arr_bool", "bools", [1, 0, 1]),
        ("arr_i32", "tokenizer.ggml.token_type", [1, -2, 3, 4])]


def test_reference_writer_file(tmp_path, writer):
    rng = np.random.default_rng(11)
    ts = _tensors(rng)
    p = str(tmp_path / "ref.gguf")
    _write(writer, p, ts, META)
    with GGUFFile(p) as g:
        assert g.version == 3 and g.alignment == 32
        hb = _header_bytes(ts, META)
        assert g.data_offset == (hb + 31) // 32 * 32
        m = g.metadata
        assert m["gemma4.block_count"] == 30 and m["neg"] == -7 and m["gemma4.rope.freq_base"] == 1.0e6
        assert m["flag"] is True and m["off"] is False and m["general.architecture"] == "gemma4"
        assert m["tokenizer.ggml.tokens"] == ["<s>", "a", "bc", ""]
        assert list(m["bytes"]) == [0, 7, 255] and list(m["shorts"]) == [-2, 3, 32767]
        assert list(m["bools"]) == [1, 0, 1] and list(m["tokenizer.ggml.token_type"]) == [1, -2, 3, 4]
        assert list(g.tensors) == [t[0] for t in ts]
        off = 0
        for name, t, dims, data in ts:
            gt = g.tensors[name]
            assert gt.type == t and gt.dims == dims
            assert gt.offset == off, name
            assert gt.nbytes == data.nbytes and np.array_equal(gt.data, data), name
            off += (data.nbytes + 31) // 32 * 32


def test_reference_writer_general_alignment_key(tmp_path, writer):
    """general.alignment read from the metadata (u32), here the writer's 32."""
    rng = np.random.default_rng(12)
    ts = _tensors(rng)[:2]
    p = str(tmp_path / "a.gguf")
    _write(writer, p, ts, [("u32", "general.alignment", 32)])
    with GGUFFile(p) as g:
        assert g.alignment == 32 and g.metadata["general.alignment"] == 32
        for name, t, dims, data in ts:
            assert np.array_equal(g.tensors[name].data, data)


def test_reference_writer_no_tensors(tmp_path, writer):
    p = str(tmp_path / "empty.gguf")
    _write(writer, p, [], [("str", "general.architecture", "none")])
    with GGUFFile(p) as g:
        assert g.tensors == {} and g.metadata["general.architecture"] == "none"


@pytest.mark.parametrize("cut", [1, 31, 200])
def test_reference_writer_truncated(tmp_path, writer, cut):
    """The writer's truncate option cuts the data section; the last tensor
    then runs past EOF and the file is rejected."""
    rng = np.random.default_rng(13)
    ts = _tensors(rng)
    p = str(tmp_path / "t.gguf")
    last = ts[-1][3].nbytes
    pad = (last + 31) // 32 * 32 - last
    _write(writer, p, ts, META, truncate=pad + cut)
    with pytest.raises(GGUFError, match="past EOF"):
        GGUFFile(p)
