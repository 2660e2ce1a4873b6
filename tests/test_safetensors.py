"""The safetensors reader (dq8_st_*, host code of libdq8.so) without a GPU.

Checked against:
  * the reference's own loader tests (weights.rs:741-799), restated;
  * the reference's tiny test checkpoints (tests/golden/tiny), read with the
    installed `safetensors` package -- version 0.8.0, the crate the reference
    pins (Cargo.lock), so its acceptance of a header is the reference's;
  * the oracle's decode restatement (dq8o.decode_weights), itself pinned by
    the reference's known answers and numpy's exact float16 conversion on all
    65536 bit patterns;
  * differential acceptance against the `safetensors` package on crafted and
    randomly generated headers.
"""
import json
import os
import struct

import numpy as np
import pytest
from hypothesis import given, settings, strategies as hst

import dq8
import dq8o

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny")


def st_file(tmp_path, header, data=b"", name="t.safetensors", size=None):
    text = header if isinstance(header, bytes) else json.dumps(header).encode()
    path = tmp_path / name
    path.write_bytes(struct.pack("<Q", len(text) if size is None else size) + text + data)
    return str(path)


def open_status(path):
    try:
        dq8.SafeTensors(path).close()
        return dq8.OK
    except dq8.Dq8Error as e:
        return e.status


def crate_accepts(path):
    """The safetensors crate's verdict on a whole file (its Python binding)."""
    import safetensors

    try:
        safetensors.deserialize(open(path, "rb").read())
        return True
    except Exception:
        return False


def crate_tensors(path):
    import safetensors

    return {name: (info["dtype"], tuple(info["shape"])) for name, info in safetensors.deserialize(open(path, "rb").read())}


# ------------------------------------------------ the reference's own tests

def test_half_and_bfloat_readout(tmp_path):
    # weights.rs:741-753: BF16 bytes 80 3f 00 c0 read as [1.0, -2.0];
    # half(0x3c00) = 1, half(0xc000) = -2, half(1) = 2^-24.
    p = st_file(tmp_path, {"w": {"dtype": "BF16", "shape": [2], "data_offsets": [0, 4]}}, bytes([0x80, 0x3F, 0x00, 0xC0]))
    with dq8.SafeTensors(p) as st:
        assert st.read_f32("w").tolist() == [1.0, -2.0]
    got = dq8o.decode_weights(np.array([0x3C00, 0xC000, 1], np.uint16), "F16")
    assert got.tolist() == [1.0, -2.0, 2.0 ** -24]
    p = st_file(tmp_path, {"w": {"dtype": "F16", "shape": [3], "data_offsets": [0, 6]}},
                np.array([0x3C00, 0xC000, 1], np.uint16).tobytes(), name="h.safetensors")
    with dq8.SafeTensors(p) as st:
        assert st.read_f32("w").tolist() == [1.0, -2.0, 2.0 ** -24]
    # Data::read of an I8 tensor: "unsupported weight dtype"
    p = st_file(tmp_path, {"w": {"dtype": "I8", "shape": [1], "data_offsets": [0, 1]}}, b"\0", name="i.safetensors")
    with dq8.SafeTensors(p) as st:
        with pytest.raises(dq8.Dq8Error) as e:
            st.read_f32("w")
        assert e.value.status == dq8.ERR_FORMAT


def test_streaming_metadata_rejects_invalid_offsets_lengths_and_values(tmp_path):
    # weights.rs:777-839
    valid = {"text.w": {"dtype": "BF16", "shape": [1], "data_offsets": [0, 2]},
             "vision.w": {"dtype": "I8", "shape": [1], "data_offsets": [2, 3]}}
    with dq8.SafeTensors(st_file(tmp_path, valid, bytes([0x80, 0x3F, 0]))) as st:
        assert st.names == ["text.w", "vision.w"]
        assert st.read_f32("text.w").tolist() == [1.0]
    assert open_status(st_file(tmp_path, valid, bytes([0x80, 0x3F]), name="a")) == dq8.ERR_FORMAT
    assert open_status(st_file(tmp_path, valid, bytes([0x80, 0x3F, 0, 0]), name="b")) == dq8.ERR_FORMAT
    with dq8.SafeTensors(st_file(tmp_path, valid, bytes([0x80, 0x7F, 0]), name="c")) as st:
        with pytest.raises(dq8.NonFinite):
            st.read_f32("text.w")
        with pytest.raises(dq8.NonFinite):
            st.read("text.w")
    gap = {"text.w": {"dtype": "BF16", "shape": [1], "data_offsets": [1, 3]}}
    assert open_status(st_file(tmp_path, gap, b"\0\0\0", name="d")) == dq8.ERR_FORMAT
    # a header size of u64::MAX
    p = tmp_path / "e"
    p.write_bytes(struct.pack("<Q", 2 ** 64 - 1))
    assert open_status(str(p)) == dq8.ERR_FORMAT
    # the 16 MiB bound (weights.rs:308) holds even inside a long enough file
    p = tmp_path / "f"
    p.write_bytes(struct.pack("<Q", (16 << 20) + 1) + b" " * ((16 << 20) + 2))
    assert open_status(str(p)) == dq8.ERR_FORMAT
    assert open_status(str(tmp_path / "missing")) == dq8.ERR_IO


# ------------------------------------------------- the reference's fixtures

@pytest.mark.parametrize("fname", ["base_model.safetensors", "adapter_model.safetensors", "head.safetensors"])
def test_reference_fixtures_read_as_the_safetensors_crate_reads_them(fname):
    from safetensors.numpy import load_file

    path = os.path.join(GOLDEN, fname)
    want = load_file(path)
    with dq8.SafeTensors(path) as st:
        assert set(st.names) == set(want)
        offsets = [t[3] for t in st.tensors]
        assert sum(offsets) == os.path.getsize(path) - 8 - struct.unpack("<Q", open(path, "rb").read(8))[0]
        for name, dt, shape, nbytes in st.tensors:
            assert dt == "F32" and shape == want[name].shape and nbytes == want[name].nbytes
            assert st.read_f32(name).tobytes() == want[name].astype(np.float32).tobytes()
            assert st.read(name).tobytes() == want[name].tobytes()
        # file order: ascending data offsets (Metadata::offset_keys)
        assert st.names == sorted(st.names, key=lambda n: crate_order(path).index(n))


def crate_order(path):
    raw = open(path, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    h = json.loads(raw[8:8 + n])
    h.pop("__metadata__", None)
    return sorted(h, key=lambda k: tuple(h[k]["data_offsets"]))


def test_projection_rule_selects_the_reference_projection_weights():
    # weights.rs:346-351 on the base checkpoint with its prefix removed
    with dq8.SafeTensors(os.path.join(GOLDEN, "base_model.safetensors")) as st:
        prefix = "model.language_model."
        proj = [n[len(prefix):] for n, _, shape, _ in st.tensors if dq8.is_projection(n[len(prefix):], shape)]
    assert sorted(proj) == sorted([
        "layers.0.linear_attn.in_proj_a.weight", "layers.0.linear_attn.in_proj_b.weight",
        "layers.0.linear_attn.in_proj_qkv.weight", "layers.0.linear_attn.in_proj_z.weight",
        "layers.0.linear_attn.out_proj.weight", "layers.0.mlp.down_proj.weight", "layers.0.mlp.gate_proj.weight",
        "layers.0.mlp.up_proj.weight", "layers.1.mlp.down_proj.weight", "layers.1.mlp.gate_proj.weight",
        "layers.1.mlp.up_proj.weight", "layers.1.self_attn.k_proj.weight", "layers.1.self_attn.o_proj.weight",
        "layers.1.self_attn.q_proj.weight", "layers.1.self_attn.v_proj.weight"])


# ------------------------------------------------------------------ decoding

def test_oracle_half_decode_is_the_ieee_conversion_on_every_pattern():
    v = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = dq8o.decode_weights(v, "F16")
    want = v.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert got[~nan].tobytes() == want[~nan].tobytes()
    assert dq8o.decode_weights(np.array([0x8000], np.uint16), "F16").view(np.uint32)[0] == 0x80000000  # -0.0


@pytest.mark.parametrize("dtype", ["BF16", "F16"])
def test_every_finite_16bit_pattern_decodes_exactly(tmp_path, dtype):
    v = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    mask = 0x7F80 if dtype == "BF16" else 0x7C00
    v = v[(v & mask) != mask]
    p = st_file(tmp_path, {"w": {"dtype": dtype, "shape": [len(v)], "data_offsets": [0, 2 * len(v)]}}, v.tobytes())
    with dq8.SafeTensors(p) as st:
        assert st.read("w").tobytes() == v.tobytes()
        assert st.read_f32("w").tobytes() == dq8o.decode_weights(v, dtype).tobytes()


@pytest.mark.parametrize("dtype,bad", [("BF16", 0x7F80), ("BF16", 0xFF81), ("F16", 0x7C00), ("F16", 0xFE01),
                                       ("F32", 0x7F800000), ("F32", 0xFFC00001)])
def test_non_finite_weights_are_rejected(tmp_path, dtype, bad):
    es = 4 if dtype == "F32" else 2
    raw = np.zeros(3000, np.uint32 if es == 4 else np.uint16)
    raw[2999] = bad
    assert not dq8o.weights_finite(raw, dtype)
    p = st_file(tmp_path, {"w": {"dtype": dtype, "shape": [3000], "data_offsets": [0, es * 3000]}}, raw.tobytes())
    with dq8.SafeTensors(p) as st:
        for read in (st.read, st.read_f32):
            with pytest.raises(dq8.NonFinite):
                read("w")


def test_bf16_and_f16_files_written_by_the_safetensors_package(tmp_path):
    import torch
    from safetensors.torch import save_file, load_file

    g = torch.Generator().manual_seed(5)
    t = {"layers.0.mlp.up_proj.weight": (torch.randn(96, 131, generator=g) * 0.05).to(torch.bfloat16),
         "layers.0.mlp.down_proj.weight": (torch.randn(131, 96, generator=g) * 3).to(torch.float16),
         "norm.weight": torch.randn(131, generator=g)}
    path = str(tmp_path / "m.safetensors")
    save_file(t, path, metadata={"format": "pt"})
    ref = load_file(path)
    with dq8.SafeTensors(path) as st:
        assert set(st.names) == set(t)
        for name, x in ref.items():
            dt, shape, _ = st.info(name)
            assert dt == {torch.bfloat16: "BF16", torch.float16: "F16", torch.float32: "F32"}[x.dtype]
            assert shape == tuple(x.shape)
            assert st.read_f32(name).tobytes() == x.float().numpy().tobytes()
            if x.dtype != torch.float32:
                assert st.read(name).tobytes() == x.view(torch.int16).numpy().tobytes()


# -------------------------------------------- acceptance vs the crate itself

F32_1 = {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}
CASES = [
    (json.dumps({"a": F32_1}).encode(), 4),
    (b' \n{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}  ', 4),  # surrounding whitespace
    (b'{"a": {"dtype": "F32", "dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}', 4),  # repeated field
    (b'{"a": {"dtype": "F32", "x": [1, {"y": -2.5e3}, null, true], "shape": [1], "data_offsets": [0, 4]}}', 4),
    (b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}, "a": {"dtype": "F32", "shape": [2], '
     b'"data_offsets": [0, 8]}}', 8),  # repeated name: the last entry
    (b'{"__metadata__": null, "a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}', 4),
    (b'{"__metadata__": {"format": "pt", "k": "\\u00e9"}, "a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}', 4),
    (b'{"__metadata__": {"x": 1}, "a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}', 4),
    (b'{"a": {"dtype": "F4", "shape": [3], "data_offsets": [0, 2]}}', 2),  # half a byte left over
    (b'{"a": {"dtype": "F4", "shape": [4], "data_offsets": [0, 2]}}', 2),
    (b'{"a": {"dtype": "F6_E2M3", "shape": [4], "data_offsets": [0, 3]}}', 3),
    (b'{"a": {"dtype": "C64", "shape": [1], "data_offsets": [0, 8]}}', 8),
    (b'{"a": {"dtype": "F8_E8M0", "shape": [2], "data_offsets": [0, 2]}}', 2),
    (b'{"a": {"dtype": "Q4", "shape": [2], "data_offsets": [0, 1]}}', 1),  # unknown dtype
    (b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4.0]}}', 4),
    (b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 04]}}', 4),
    (b'{"a": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}', 4),
    (b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4, 8]}}', 8),
    (b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0]}}', 4),
    (b'{"a": {"dtype": "F32", "shape": [1]}}', 4),  # missing field
    (json.dumps({"a": F32_1}).encode() + b" x", 4),  # trailing text
    (json.dumps({"a": F32_1}).encode(), 5),  # data past the last tensor
    (json.dumps({"a": F32_1}).encode(), 3),
    (b'{}', 0),
    (b'[]', 0),
    (b'{"\\ud83d\\ude00": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}', 1),  # surrogate pair
    (b'{"\\ud83d": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}', 1),  # lone surrogate
    (b'{"\xc3\xa9": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}', 1),  # UTF-8 name
    (b'{"\xc3": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}', 1),  # broken UTF-8
    (b'{"a\x01": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}', 1),  # control character
    (b'{"a": {"dtype": "U8", "shape": [2, 0], "data_offsets": [0, 0]}, "b": {"dtype": "U8", "shape": [], '
     b'"data_offsets": [0, 1]}}', 1),  # empty tensor, scalar
    (b'{"a": {"dtype": "U8", "shape": [18446744073709551615, 2], "data_offsets": [0, 1]}}', 1),  # overflow
    (b'{"a": {"dtype": "U8", "shape": [1], "data_offsets": [1, 2]}, "b": {"dtype": "U8", "shape": [1], '
     b'"data_offsets": [0, 1]}}', 2),  # out of order in the text
    (b'{"a": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]}, "b": {"dtype": "U8", "shape": [1], '
     b'"data_offsets": [1, 2]}}', 2),  # overlap
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_header_acceptance_matches_the_safetensors_crate(tmp_path, case):
    header, data_len = CASES[case]
    path = st_file(tmp_path, header, b"\0" * data_len)
    ours = open_status(path)
    assert ours in (dq8.OK, dq8.ERR_FORMAT)
    assert (ours == dq8.OK) == crate_accepts(path), header
    if ours == dq8.OK:
        with dq8.SafeTensors(path) as st:
            assert {n: (d, s) for n, d, s, _ in st.tensors} == crate_tensors(path)


DTYPES = ["F32", "BF16", "F16", "I8", "U8", "F64", "I64", "BOOL", "F8_E4M3", "F4", "F6_E3M2", "C64", "X9"]

BITS = {"F32": 32, "BF16": 16, "F16": 16, "I8": 8, "U8": 8, "F64": 64, "I64": 64, "BOOL": 8, "F8_E4M3": 8, "F4": 4,
        "F6_E3M2": 6, "C64": 64, "X9": 8}

tensor_entry = hst.fixed_dictionaries({
    "name": hst.text(alphabet="abc.\u00e9_", min_size=1, max_size=4),
    "dtype": hst.sampled_from(DTYPES),
    "shape": hst.lists(hst.integers(0, 5), max_size=3),
    "skew": hst.sampled_from([0, 0, 0, 0, 1, -1, 2]),
    "extra": hst.booleans(),
})


@settings(max_examples=300, deadline=None)
@given(entries=hst.lists(tensor_entry, max_size=5), shuffle=hst.randoms(), tail=hst.sampled_from([0, 0, 0, 1, -1]),
       meta=hst.sampled_from([None, {"format": "pt"}, "null"]))
def test_random_headers_are_accepted_exactly_when_the_crate_accepts_them(tmp_path_factory, entries, shuffle, tail,
                                                                        meta):
    header, start = {}, 0
    for e in entries:
        nbytes = (int(np.prod(e["shape"], dtype=np.int64)) * BITS[e["dtype"]] + 7) // 8
        begin = max(0, start + e["skew"])
        info = {"dtype": e["dtype"], "shape": e["shape"], "data_offsets": [begin, begin + nbytes]}
        if e["extra"]:
            info["note"] = [1, "x", {"y": None}]
        header[e["name"]] = info
        start = begin + nbytes
    items = list(header.items())
    shuffle.shuffle(items)
    text = "{" + ", ".join(json.dumps(k) + ": " + json.dumps(v) for k, v in items)
    if meta is not None:
        text += (", " if items else "") + '"__metadata__": ' + (meta if meta == "null" else json.dumps(meta))
    text += "}"
    data_len = max(0, max([v["data_offsets"][1] for v in header.values()] or [0]) + tail)
    path = st_file(tmp_path_factory.mktemp("h"), text.encode(), b"\0" * data_len)
    ours = open_status(path)
    assert ours in (dq8.OK, dq8.ERR_FORMAT)
    assert (ours == dq8.OK) == crate_accepts(path), text
    if ours == dq8.OK:
        with dq8.SafeTensors(path) as f:
            assert {n: (d, sh) for n, d, sh, _ in f.tensors} == crate_tensors(path)


BASE = (b'{"__metadata__": {"format": "pt"}, "w.a": {"dtype": "BF16", "shape": [2, 3], "data_offsets": [0, 12]}, '
        b'"w.b": {"dtype": "F32", "shape": [1], "data_offsets": [12, 16]}}')


@settings(max_examples=300, deadline=None)
@given(pos=hst.integers(0, len(BASE) - 1), byte=hst.integers(0, 255), op=hst.sampled_from(["set", "insert", "delete"]))
def test_mutated_headers_are_accepted_exactly_when_the_crate_accepts_them(tmp_path_factory, pos, byte, op):
    b = bytearray(BASE)
    if op == "set":
        b[pos] = byte
    elif op == "insert":
        b.insert(pos, byte)
    else:
        del b[pos]
    path = st_file(tmp_path_factory.mktemp("m"), bytes(b), b"\0" * 16)
    ours = open_status(path)
    assert ours in (dq8.OK, dq8.ERR_FORMAT)
    assert (ours == dq8.OK) == crate_accepts(path), bytes(b)
    if ours == dq8.OK:
        with dq8.SafeTensors(path) as f:
            assert {n: (d, sh) for n, d, sh, _ in f.tensors} == crate_tensors(path)
