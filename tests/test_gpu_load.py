"""GPU parity of the weight load path: stored F32/BF16/F16 elements -> device
decode -> Data::quantize -> repack, from device memory (dq8_weights_from_raw),
host memory (dq8_weights_upload) and safetensors files (dq8_st_load_weights).
The exported Data::Quantized must equal the oracle's quantization of the
oracle's decoding (dq8o.decode_weights), bit for bit."""
import json
import os
import struct

import numpy as np
import pytest
import torch

import dq8
import dq8o

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny")
DTYPE = {"F32": dq8.F32, "BF16": dq8.BF16, "F16": dq8.F16}


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def exported(w):
    v, s = w.export()
    return host(v), host(s)


def expect(raw, dtype):
    return dq8o.quantize_weights(dq8o.decode_weights(raw, dtype))


def assert_same(w, raw, dtype):
    v, s = exported(w)
    ev, es = expect(raw, dtype)
    assert np.array_equal(v, ev)
    assert s.tobytes() == es.tobytes()


def random_raw(rng, n, k, dtype, scale=0.05):
    x = (rng.standard_normal((n, k)) * scale).astype(np.float32)
    x[0, : min(k, 5)] = [0.0, -0.0, 1e-40, -3e-39, 6e4][: min(k, 5)]  # zeros and subnormals
    if dtype == "F32":
        return x
    t = torch.from_numpy(x).to(torch.bfloat16 if dtype == "BF16" else torch.float16)
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def write_st(path, tensors):
    """A safetensors file of raw arrays: {name: (dtype, ndarray of stored elements)}."""
    header, blobs, off = {}, [], 0
    for name, (dt, a) in tensors.items():
        b = np.ascontiguousarray(a).tobytes()
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    text = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)) + text + b"".join(blobs))


def test_reference_fixture_projections_load_bit_exact(ctx):
    prefix = "model.language_model."
    with dq8.SafeTensors(os.path.join(GOLDEN, "base_model.safetensors")) as st:
        names = [n for n, _, shape, _ in st.tensors if dq8.is_projection(n[len(prefix):], shape)]
        assert len(names) == 15
        for name in names:
            w = st.load_weights(ctx, name)
            assert_same(w, st.read(name), "F32")
            w.free()


@pytest.mark.parametrize("dtype", ["F32", "BF16", "F16"])
@pytest.mark.parametrize("n,k", [(1, 1), (31, 131), (256, 2048), (97, 4160)])
def test_raw_weights_from_device_and_host_match_the_oracle(ctx, dtype, n, k):
    rng = np.random.default_rng(n * 7 + k + len(dtype))
    raw = random_raw(rng, n, k, dtype)
    dev = torch.from_numpy(raw.view(np.int16) if dtype != "F32" else raw).cuda()
    if dtype == "BF16":
        dev = dev.view(torch.bfloat16)
    elif dtype == "F16":
        dev = dev.view(torch.float16)
    w1 = ctx.weights_from_raw(dev)
    w2 = ctx.weights_upload(raw, DTYPE[dtype])
    assert_same(w1, raw, dtype)
    assert_same(w2, raw, dtype)


@pytest.mark.parametrize("dtype", ["BF16", "F16"])
def test_every_finite_16bit_pattern_quantizes_as_the_oracle(ctx, dtype):
    # All finite bit patterns, 64 to a group; once in order, once shuffled so
    # that every group mixes magnitudes.
    v = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    mask = 0x7F80 if dtype == "BF16" else 0x7C00
    v = v[(v & mask) != mask]
    v = np.concatenate([v, np.random.default_rng(1).permutation(v)])
    v = v[: len(v) // 2048 * 2048].reshape(-1, 2048)
    w = ctx.weights_upload(np.ascontiguousarray(v), DTYPE[dtype])
    assert_same(w, v, dtype)


def test_large_file_streams_through_the_staging_buffers(ctx, tmp_path):
    # 8224 x 2048 BF16 (33.7 MB: five 8 MiB staging slices) and a ragged F16
    # tensor behind it in the same file.
    rng = np.random.default_rng(8224)
    a = random_raw(rng, 8224, 2048, "BF16")
    b = random_raw(rng, 333, 1000, "F16", scale=2.0)
    path = str(tmp_path / "big.safetensors")
    write_st(path, {"layers.0.linear_attn.in_proj_qkvz.weight": ("BF16", a), "layers.0.mlp.x_proj.weight": ("F16", b)})
    with dq8.SafeTensors(path) as st:
        wa = st.load_weights(ctx, "layers.0.linear_attn.in_proj_qkvz.weight")
        wb = st.load_weights(ctx, "layers.0.mlp.x_proj.weight")
        assert_same(wa, a, "BF16")
        assert_same(wb, b, "F16")
        # the loaded weights drive a projection bit-exactly
        x = rng.standard_normal((24, 2048)).astype(np.float32)
        q, s = ctx.quantize(torch.from_numpy(x).cuda())
        ev, es = expect(a, "BF16")
        assert host(ctx.linear(wa, q, s)).tobytes() == dq8o.linear(x, ev, es, threads=8).tobytes()


@pytest.mark.parametrize("dtype,bad", [("BF16", 0x7F80), ("BF16", 0xFFC1), ("F16", 0xFC00), ("F16", 0x7E00),
                                       ("F32", 0xFF800000), ("F32", 0x7FC00000)])
def test_non_finite_weights_are_rejected_on_the_device(ctx, tmp_path, dtype, bad):
    rng = np.random.default_rng(3)
    raw = random_raw(rng, 70, 300, dtype)
    if dtype == "F32":
        raw.view(np.uint32)[69, 299] = bad
    else:
        raw[69, 299] = bad
    assert not dq8o.weights_finite(raw.view(np.uint32) if dtype == "F32" else raw, dtype)
    with pytest.raises(dq8.NonFinite):
        ctx.weights_upload(raw, DTYPE[dtype])
    dev = torch.from_numpy(raw.view(np.int16) if dtype != "F32" else raw).cuda()
    dev = dev.view({"BF16": torch.bfloat16, "F16": torch.float16}.get(dtype, torch.float32))
    with pytest.raises(dq8.NonFinite):
        ctx.weights_from_raw(dev)
    path = str(tmp_path / "bad.safetensors")
    write_st(path, {"layers.0.mlp.up_proj.weight": (dtype, raw)})
    with dq8.SafeTensors(path) as st:
        with pytest.raises(dq8.NonFinite):
            st.load_weights(ctx, "layers.0.mlp.up_proj.weight")
    # the context keeps working after a rejected load
    ok = random_raw(rng, 5, 64, dtype)
    assert_same(ctx.weights_upload(ok, DTYPE[dtype]), ok, dtype)


def test_load_weights_rejects_non_projection_shapes_and_dtypes(ctx, tmp_path):
    path = str(tmp_path / "m.safetensors")
    write_st(path, {"a": ("F32", np.zeros((4,), np.float32)), "b": ("I8", np.zeros((2, 2), np.int8)),
                    "c": ("F32", np.zeros((3, 0), np.float32))})
    with dq8.SafeTensors(path) as st:
        for name, status in (("a", dq8.ERR_SHAPE), ("b", dq8.ERR_FORMAT), ("c", dq8.ERR_SHAPE)):
            with pytest.raises(dq8.Dq8Error) as e:
                st.load_weights(ctx, name)
            assert e.value.status == status
