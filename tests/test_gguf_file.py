"""GGUF parser / writer tests (CPU).

* A header packed by hand here with ``struct`` (independent of the writer)
  parses to the values put in, for every KV value type.
* The reference's own fixtures (``webgpu/test-fixtures/gguf-*.json``, written by
  llama.cpp's gguf-py from three real model files) pin the tensor-table math:
  for every one of their 1880 tensors, a header carrying the fixture's table
  parses to gguf-py's byte count, element count, dims, type, and offset from
  the data section, as ``webgpu/scripts/test-gguf.mts:44-62`` checks the
  reference parser.  The fixtures also pin the data layout the writer uses:
  each tensor starts at the 32-byte-aligned end of the previous one.
* Error paths keep the reference's messages (``webgpu/src/model/gguf.ts``).
"""
import importlib
import json
import os
import struct

import numpy as np
import pytest

gf = importlib.import_module("artifex-assistantv5_amd.gguf_file")
ggml = importlib.import_module("artifex-assistantv5_amd.ggml")

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _reader(buf: bytes):
    calls = []

    def read(a, b):
        calls.append((a, b))
        return buf[a:b]
    return read, calls


def _hand_header(alignment=None):
    kv = [
        (_s("general.architecture") + struct.pack("<I", 8) + _s("llama")),
        (_s("u8") + struct.pack("<IB", 0, 200)),
        (_s("i8") + struct.pack("<Ib", 1, -5)),
        (_s("u16") + struct.pack("<IH", 2, 60000)),
        (_s("i16") + struct.pack("<Ih", 3, -30000)),
        (_s("u32") + struct.pack("<II", 4, 4000000000)),
        (_s("i32") + struct.pack("<Ii", 5, -2000000000)),
        (_s("f32") + struct.pack("<If", 6, 0.25)),
        (_s("flag") + struct.pack("<IB", 7, 1)),
        (_s("u64") + struct.pack("<IQ", 10, 2 ** 40)),
        (_s("i64") + struct.pack("<Iq", 11, -(2 ** 41))),
        (_s("f64") + struct.pack("<Id", 12, 1e-300)),
        (_s("arr") + struct.pack("<IIQ", 9, 5, 3) + struct.pack("<iii", 1, -2, 3)),
        (_s("strs") + struct.pack("<IIQ", 9, 8, 2) + _s("ab") + _s("")),
    ]
    if alignment:
        kv.append(_s("general.alignment") + struct.pack("<II", 4, alignment))
    tensors = [
        _s("w") + struct.pack("<I", 2) + struct.pack("<QQ", 512, 3) + struct.pack("<IQ", 12, 0),
        _s("n") + struct.pack("<I", 1) + struct.pack("<Q", 7) + struct.pack("<IQ", 0, 896),
    ]
    head = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kv))
    return head + b"".join(kv) + b"".join(tensors)


@pytest.mark.parametrize("alignment", [None, 64])
def test_hand_packed_header(alignment):
    buf = _hand_header(alignment)
    read, _ = _reader(buf)
    f = gf.parse_gguf(read)
    assert f.version == 3 and f.tensor_count == 2
    assert f.kv["general.architecture"] == "llama"
    assert (f.kv["u8"], f.kv["i8"], f.kv["u16"], f.kv["i16"]) == (200, -5, 60000, -30000)
    assert (f.kv["u32"], f.kv["i32"]) == (4000000000, -2000000000)
    assert f.kv["f32"] == 0.25 and f.kv["flag"] is True and f.kv["f64"] == 1e-300
    assert (f.kv["u64"], f.kv["i64"]) == (2 ** 40, -(2 ** 41))
    assert f.kv["arr"] == [1, -2, 3] and f.kv["strs"] == ["ab", ""]
    align = alignment or 32
    assert f.alignment == align and f.header_bytes == len(buf)
    assert f.data_offset == -(-len(buf) // align) * align and f.data_offset % align == 0
    w, n = f.tensors["w"], f.tensors["n"]
    assert (w.ne, w.shape, w.ggml_type, w.type_name) == ([512, 3], [3, 512], 12, "Q4_K")
    assert (w.offset, w.byte_length, w.element_count) == (f.data_offset, 2 * 144 * 3, 1536)
    assert (n.offset, n.byte_length, n.element_count) == (f.data_offset + 896, 28, 7)
    assert gf.gguf_architecture(f) == "llama"
    assert gf.arch_kv(f, "missing", 7) == 7
    with pytest.raises(ValueError, match=r"Missing KV llama\.missing"):
        gf.arch_kv(f, "missing")


def test_header_grows_past_initial_fetch(monkeypatch):
    monkeypatch.setattr(gf, "INITIAL_FETCH", 64)
    kv = _s("tokens") + struct.pack("<IIQ", 9, 8, 300) + b"".join(_s(f"t{i}") for i in range(300))
    buf = struct.pack("<IIQQ", 0x46554747, 2, 0, 1) + kv
    read, calls = _reader(buf)
    f = gf.parse_gguf(read)
    assert f.kv["tokens"][299] == "t299" and f.version == 2
    assert calls[0] == (0, 64) and len(calls) > 2          # doubled on demand
    for (a0, b0), (a1, b1) in zip(calls[1:], calls[2:]):
        assert a1 == b0 and b1 == 2 * b0                    # contiguous, doubling


def _with(buf: bytes, at: int, new: bytes) -> bytes:
    return buf[:at] + new + buf[at + len(new):]


def test_errors_keep_reference_messages():
    buf = _hand_header()
    r = lambda b: _reader(b)[0]  # noqa: E731
    with pytest.raises(ValueError, match="Bad magic 0x46554746"):
        gf.parse_gguf(r(_with(buf, 0, struct.pack("<I", 0x46554746))))
    for v in (1, 4):
        with pytest.raises(ValueError, match=f"Unsupported version {v}"):
            gf.parse_gguf(r(_with(buf, 4, struct.pack("<I", v))))
    with pytest.raises(ValueError, match="exceeds safe integer"):
        gf.parse_gguf(r(_with(buf, 8, struct.pack("<Q", 2 ** 53))))
    bad_kv = struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + _s("k") + struct.pack("<I", 13)
    with pytest.raises(ValueError, match="Unknown KV value type 13"):
        gf.parse_gguf(r(bad_kv))
    dims5 = (struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + _s("t") + struct.pack("<I", 5)
             + struct.pack("<5Q", 1, 1, 1, 1, 1) + struct.pack("<IQ", 0, 0))
    with pytest.raises(ValueError, match='Tensor "t" has 5 dims'):
        gf.parse_gguf(r(dims5))
    badtype = (struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + _s("t") + struct.pack("<I", 1)
               + struct.pack("<Q", 32) + struct.pack("<IQ", 4, 0))
    with pytest.raises(ggml.GGMLTypeError, match="Unsupported ggml type 4"):
        gf.parse_gguf(r(badtype))
    ragged = (struct.pack("<IIQQ", 0x46554747, 3, 1, 0) + _s("t") + struct.pack("<I", 1)
              + struct.pack("<Q", 100) + struct.pack("<IQ", 12, 0))
    with pytest.raises(ValueError, match=r"ne\[0\]=100 not divisible by block size 256"):
        gf.parse_gguf(r(ragged))
    with pytest.raises(ValueError, match="Short read growing header buffer"):
        gf.parse_gguf(r(buf[:-3]))


def _tables():
    with open(os.path.join(GOLDEN, "gguf_tensor_tables.json"), encoding="utf-8") as f:
        return json.load(f)["files"]


@pytest.mark.parametrize("fx", _tables(), ids=lambda fx: fx["source"].split("/")[-1])
def test_reference_fixture_tensor_tables(fx):
    tensors = fx["tensors"]
    assert len(tensors) == fx["tensor_count"]
    assert fx["data_offset"] % fx["alignment"] == 0
    # the files lay tensors out back to back, each at the aligned end of the last
    rel = [t[3] - fx["data_offset"] for t in tensors]
    order = sorted(range(len(tensors)), key=lambda i: rel[i])
    pos = 0
    for i in order:
        assert rel[i] == pos, tensors[i][0]
        pos += -(-tensors[i][4] // fx["alignment"]) * fx["alignment"]
    # a header carrying the fixture's table parses to gguf-py's numbers
    kv = {"general.architecture": fx["kv"]["general.architecture"], **fx["kv"]}
    kv_types = {k: gf.GGUFValueType.FLOAT64 for k, v in kv.items() if isinstance(v, float)}
    table = [(t[0], t[1], t[2], t[4]) for t in (tensors[i] for i in order)]
    head, offs = gf.gguf_header_bytes(kv, table, alignment=fx["alignment"], kv_types=kv_types)
    assert offs == [rel[i] for i in order]
    f = gf.parse_gguf(_reader(head)[0])
    assert (f.version, f.tensor_count, f.alignment) == (fx["version"], fx["tensor_count"],
                                                        fx["alignment"])
    for name, ne, typ, abs_off, nbytes, nel in tensors:
        t = f.tensors[name]
        assert (t.ne, t.ggml_type, t.byte_length, t.element_count) == (ne, typ, nbytes, nel), name
        assert t.offset - f.data_offset == abs_off - fx["data_offset"], name
        assert t.byte_length == ggml.ggml_tensor_bytes(typ, ne)
    for k, v in fx["kv"].items():
        assert f.kv[k] == v, k


def test_writer_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    tensors = [("a.weight", [64, 3], 0, rng.standard_normal(192).astype(np.float32)),
               ("b.weight", [256, 5], 12, rng.integers(0, 256, 5 * 144, dtype=np.uint8)),
               ("c.weight", [32, 2], 8, rng.integers(0, 256, 2 * 34, dtype=np.uint8)),
               ("d.weight", [256, 1], 14, rng.integers(0, 256, 210, dtype=np.uint8))]
    p = str(tmp_path / "m.gguf")
    gf.write_gguf(p, {"general.architecture": "llama", "llama.block_count": 1,
                      "llama.rope.freq_base": 5e5, "names": ["x", "y"]}, tensors,
                  alignment=64)
    f = gf.parse_gguf_path(p)
    assert f.alignment == 64 and f.kv["llama.rope.freq_base"] == 5e5
    assert f.kv["names"] == ["x", "y"]
    size = os.path.getsize(p)
    for name, ne, typ, data in tensors:
        t = f.tensors[name]
        assert t.offset % 64 == 0 and t.offset + t.byte_length <= size
        got = np.asarray(gf.map_tensor_bytes(p, t))
        assert got.tobytes() == data.tobytes()
    with pytest.raises(ValueError, match="needs 288"):
        gf.write_gguf(p, {}, [("x", [256, 2], 12, np.zeros(287, np.uint8))])


def test_loader_preflight_runs_before_any_device_work(tmp_path):
    """Unsupported types, an HBM budget overrun, another architecture or a tensor
    the llama decoder has no slot for all raise before a byte is placed
    (gguf-loader.ts:229-256)."""
    import gguf_models as gm
    loader = importlib.import_module("artifex-assistantv5_amd.gguf_loader")
    gmodel = importlib.import_module("artifex-assistantv5_amd.gguf_model")
    tensors = gm.make_model(seed=1)
    p = str(tmp_path / "q41.gguf")
    gm.write_model(p, tensors, extra_tensors=[
        ("blk.0.odd.weight", [32, 2], 3, np.zeros(40, np.uint8)),
        ("blk.1.odd.weight", [32, 2], 3, np.zeros(40, np.uint8))])
    with pytest.raises(ValueError, match=r"can't run yet: Q4_1 \(2 tensors\)"):
        loader.load_gguf_model(p, "cuda")
    p2 = str(tmp_path / "ok.gguf")
    gm.write_model(p2, tensors)
    with pytest.raises(ValueError, match="budget is 0.00 GB"):
        loader.load_gguf_model(p2, "cuda", vram_budget_bytes=1000)
    p3 = str(tmp_path / "qwen.gguf")
    gm.write_model(p3, tensors, extra_kv={"general.architecture": "qwen3"})
    with pytest.raises(NotImplementedError, match="architecture 'qwen3'"):
        gmodel.load_decoder(p3, "cuda")
    p4 = str(tmp_path / "bias.gguf")
    gm.write_model(p4, tensors, extra_tensors=[
        ("blk.0.attn_q.bias", [256], 0, np.zeros(256, np.float32))])
    with pytest.raises(NotImplementedError, match="no slot for 1 tensor"):
        gmodel.load_decoder(p4, "cuda")


def test_unpermute_inverts_the_converter_permutation():
    import gguf_models as gm
    gmodel = importlib.import_module("artifex-assistantv5_amd.gguf_model")
    for nh, hd in ((4, 64), (2, 128), (1, 8)):
        orig = np.arange(nh * hd)
        stored = orig[gm.permute_rows(nh, hd)]
        assert np.array_equal(stored[gmodel.unpermute_rows(nh, hd)], orig)
        # the converter's rule: stored row h*hd + 2j + p is original row h*hd + p*hd/2 + j
        assert stored[1] == hd // 2 and stored[2] == 1
