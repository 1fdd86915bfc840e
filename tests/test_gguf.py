"""GGUF reader (laplace_amd.gguf, following GGUFContext::open,
src/gguf.cpp:209-389) on files written by laplace_amd.gguf.write_gguf:
metadata value types, tensor infos, alignment and data offsets, bounds
checks; and, on the GPU, the host-pointer matmul entries on a registered
file's tensors (device residency, src/matmul.cpp:446-448)."""
import os
import struct

import numpy as np
import pytest

from laplace_amd.gguf import GGUFError, GGUFFile, tensor_nbytes, write_gguf

Q8_0, Q4_K, Q6_K, F32 = 8, 12, 14, 0


def _tensors(rng):
    return [("blk.0.attn_q.weight", Q4_K, (512, 24), rng.integers(0, 256, tensor_nbytes(Q4_K, (512, 24)), dtype=np.uint8)),
            ("blk.0.ffn_down.weight", Q6_K, (256, 7), rng.integers(0, 256, tensor_nbytes(Q6_K, (256, 7)), dtype=np.uint8)),
            ("output_norm.weight", F32, (33,), rng.standard_normal(33).astype(np.float32).view(np.uint8)),
            ("token_embd.weight", Q8_0, (64, 5), rng.integers(0, 256, tensor_nbytes(Q8_0, (64, 5)), dtype=np.uint8))]


@pytest.mark.parametrize("alignment", [32, 64, 4096])
def test_round_trip(tmp_path, alignment):
    rng = np.random.default_rng(alignment)
    ts = _tensors(rng)
    meta = {"general.architecture": "gemma4", "gemma4.block_count": np.uint32(30), "big": 2 ** 40,
            "gemma4.rope.freq_base": 1e6, "flag": True, "tokenizer.ggml.tokens": ["<s>", "a", "bc"],
            "i8": np.int8(-3), "u16": np.uint16(7), "i64": np.int64(-9), "f64": np.float64(0.25),
            "scores": np.arange(5, dtype=np.float32), "types": np.array([1, -2, 3], np.int32)}
    p = str(tmp_path / "m.gguf")
    write_gguf(p, ts, meta, alignment=alignment)
    with GGUFFile(p) as g:
        assert g.version == 3 and g.alignment == alignment
        assert g.data_offset % alignment == 0
        m = g.metadata
        assert m["general.architecture"] == "gemma4" and m["gemma4.block_count"] == 30
        assert m["big"] == 2 ** 40 and m["flag"] is True and m["i8"] == -3 and m["u16"] == 7
        assert m["i64"] == -9 and m["f64"] == 0.25 and abs(m["gemma4.rope.freq_base"] - 1e6) < 1
        assert m["tokenizer.ggml.tokens"] == ["<s>", "a", "bc"]
        assert np.array_equal(m["scores"], np.arange(5, dtype=np.float32))
        assert np.array_equal(m["types"], [1, -2, 3])
        assert list(g.tensors) == [t[0] for t in ts]
        for name, t, dims, data in ts:
            gt = g.tensors[name]
            assert gt.type == t and gt.dims == dims and gt.offset % alignment == 0
            assert gt.nbytes == data.nbytes and np.array_equal(gt.data, data)
        assert g.find_tensor("nope") is None
        assert g.find_tensor("blk.0.attn_q.weight").dims == (512, 24)


def test_errors(tmp_path):
    rng = np.random.default_rng(1)
    p = str(tmp_path / "m.gguf")
    write_gguf(p, _tensors(rng), {"a": "b"})
    raw = open(p, "rb").read()

    def bad(data, what):
        q = str(tmp_path / "bad.gguf")
        open(q, "wb").write(data)
        with pytest.raises(GGUFError, match=what):
            GGUFFile(q)

    bad(b"GGUX" + raw[4:], "bad magic")
    bad(raw[:4] + struct.pack("<I", 4) + raw[8:], "unsupported version")
    bad(raw[:30], "past EOF")
    bad(raw[:-10], "past EOF")            # last tensor's data cut short
    q = str(tmp_path / "empty.gguf")
    open(q, "wb").close()
    with pytest.raises(GGUFError):
        GGUFFile(q)


def test_version_2_and_default_alignment(tmp_path):
    rng = np.random.default_rng(2)
    p = str(tmp_path / "v2.gguf")
    write_gguf(p, _tensors(rng)[:1], {}, version=2)
    with GGUFFile(p) as g:
        assert g.version == 2 and g.alignment == 32 and "general.alignment" not in g.metadata


REF_FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_writer_weights.gguf")


def _own_writer_file(tmp_path):
    from hip_util import synth_weights
    K, N = 1024, 96
    ws = [("q4k", Q4_K, synth_weights(Q4_K, K, N, seed=1)), ("q6k", Q6_K, synth_weights(Q6_K, K, N, seed=2)),
          ("q80", Q8_0, synth_weights(Q8_0, K, N, seed=3))]
    p = str(tmp_path / "w.gguf")
    write_gguf(p, [(n, t, (K, N), w) for n, t, w in ws], {"general.architecture": "test"})
    return p


def test_reference_fixture_reads():
    """The committed fixture written by the reference's writer
    (tests/golden/make_gguf_fixture.py) parses: three K 1024 x N 32 tensors."""
    with GGUFFile(REF_FIXTURE) as g:
        assert g.version == 3 and g.metadata["general.architecture"] == "laplace-test"
        assert {n: (t.type, t.dims) for n, t in g.tensors.items()} == {
            "w.q4k": (Q4_K, (1024, 32)), "w.q6k": (Q6_K, (1024, 32)), "w.q80": (Q8_0, (1024, 32))}


@pytest.mark.gpu
@pytest.mark.parametrize("which", ["own_writer", "reference_writer"])
def test_registered_file_matmul(tmp_path, orc, which):
    """The reference's flow: mmap the GGUF, register the data region once,
    then call the back-end with host weight pointers into the mapping. Run
    on a file from write_gguf and on the committed fixture written by the
    reference's own writer (tests/gguf_writer.h)."""
    from hip_util import synth_x
    from laplace_amd._lib import lib
    p = _own_writer_file(tmp_path) if which == "own_writer" else REF_FIXTURE
    with GGUFFile(p) as g:
        K = next(iter(g.tensors.values())).dims[0]
        x = synth_x(3, K, seed=4)
        g.register()
        for name, gt in g.tensors.items():
            t, N = gt.type, gt.dims[1]
            wt = gt.data
            y = np.zeros((3, N), np.float32)
            assert lib().lp_gemm(x.ctypes.data, wt.ctypes.data, t, y.ctypes.data, 3, K, N), lib().lp_last_error()
            ref = orc.gemm_int(t, x, np.array(wt), N)
            assert np.abs(y - ref).max() <= 1e-4 * np.abs(ref).max(), name
