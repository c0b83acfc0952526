"""Safetensors weights into device memory (the reference's weight loader,
nemotron-model/src/weights.rs): header parsing and validation on the CPU,
device reads and an int8 linear layer loaded from a file on the GPU."""
import ctypes as C
import json
import os
import struct
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "nemotron-cutile-rs_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import nemotron_hip as NH  # noqa: E402
import oracle_ctypes as O  # noqa: E402
from tiling import tile_16x64  # noqa: E402


def write_file(path, tensors, header_override=None, raw_header=None):
    """The reference test writer (weights.rs:499-525): entries in order, data
    offsets relative to the data section, 8-byte little-endian header length."""
    header, data, offset = {}, b"", 0
    for name, dtype, shape, payload in tensors:
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [offset, offset + len(payload)]}
        offset += len(payload)
        data += bytes(payload)
    if header_override:
        header.update(header_override)
    hb = raw_header if raw_header is not None else json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + data)


def info(path, name):
    ti = NH.TensorInfo()
    st, err = NH.call_status("nh_safetensors_tensor_info", str(path).encode(), name.encode(), C.byref(ti))
    return st, err, ti


def test_reference_single_file_manifest_and_tensor(tmp_path):
    # weights.rs:533-565
    p = tmp_path / "model.safetensors"
    write_file(p, [("embed.weight", "F32", [2], [1, 2, 3, 4, 5, 6, 7, 8]), ("lm_head.weight", "U8", [3], [9, 10, 11])])
    st, _, ti = info(p, "embed.weight")
    assert st == NH.OK and ti.dtype == b"F32" and ti.ndim == 1 and ti.shape[0] == 2 and ti.data_bytes == 8
    hlen = struct.unpack("<Q", open(p, "rb").read(8))[0]
    assert ti.data_begin == 8 + hlen + 0
    st, _, ti = info(p, "lm_head.weight")
    assert st == NH.OK and ti.dtype == b"U8" and list(ti.shape[:ti.ndim]) == [3]
    raw = open(p, "rb").read()
    assert list(raw[ti.data_begin:ti.data_begin + ti.data_bytes]) == [9, 10, 11]


def test_reference_missing_tensor(tmp_path):
    # weights.rs:620-631: "tensor not found: missing"
    p = tmp_path / "model.safetensors"
    write_file(p, [("x", "U8", [1], [1])])
    st, err, _ = info(p, "missing")
    assert st == NH.TENSOR_NOT_FOUND and err.message.decode() == "tensor not found: missing"


def test_missing_file_is_an_io_error(tmp_path):
    st, _, _ = info(tmp_path / "nope.safetensors", "x")
    assert st == NH.IO_ERROR


@pytest.mark.parametrize("entry,reason", [
    (7, "tensor entry must be an object"),
    ({"shape": [1], "data_offsets": [0, 1]}, "missing dtype"),
    ({"dtype": "U8", "data_offsets": [0, 1]}, "missing shape"),
    ({"dtype": "U8", "shape": [-1], "data_offsets": [0, 1]}, "shape entries must be unsigned integers"),
    ({"dtype": "U8", "shape": [1.5], "data_offsets": [0, 1]}, "shape entries must be unsigned integers"),
    ({"dtype": "U8", "shape": [1]}, "missing data_offsets"),
    ({"dtype": "U8", "shape": [1], "data_offsets": [0]}, "data_offsets must contain [start, end]"),
    ({"dtype": "U8", "shape": [1], "data_offsets": ["0", 1]}, "data_offsets start must be an unsigned integer"),
    ({"dtype": "U8", "shape": [1], "data_offsets": [0, -1]}, "data_offsets end must be an unsigned integer"),
    ({"dtype": "U8", "shape": [1], "data_offsets": [1, 0]},
     "data_offsets end must be greater than or equal to start"),
])
def test_invalid_tensor_headers_use_the_reference_reasons(tmp_path, entry, reason):
    # RawTensorHeader::from_value (weights.rs:276-358); any invalid entry fails the file
    p = tmp_path / "bad.safetensors"
    write_file(p, [("good", "U8", [1], [1])], header_override={"broken": entry})
    st, err, _ = info(p, "good")
    assert st == NH.INVALID_HEADER
    assert err.message.decode().endswith(reason) and "broken" in err.message.decode()


def test_header_length_past_the_file_and_bad_json(tmp_path):
    p = tmp_path / "len.safetensors"
    with open(p, "wb") as f:
        f.write(struct.pack("<Q", 1000) + b"{}")
    st, err, _ = info(p, "x")  # InvalidHeaderLength (weights.rs:258-264)
    assert st == NH.INVALID_HEADER and (err.expected, err.actual) == (10, 1000)
    q = tmp_path / "json.safetensors"
    write_file(q, [], raw_header=b'{"x": {"dtype": "U8", ')
    assert info(q, "x")[0] == NH.INVALID_HEADER  # InvalidHeaderJson
    r = tmp_path / "arr.safetensors"
    write_file(r, [], raw_header=b"[1, 2]")
    assert info(r, "x")[0] == NH.INVALID_HEADER  # the header must be an object


def test_metadata_and_escaped_names(tmp_path):
    p = tmp_path / "meta.safetensors"
    write_file(p, [("layer.é\\n", "BF16", [2, 3], bytes(12))],
               header_override={"__metadata__": {"format": "pt"}})
    st, _, ti = info(p, "layer.é\\n")
    assert st == NH.OK and ti.dtype == b"BF16" and list(ti.shape[:2]) == [2, 3] and ti.data_bytes == 12
    assert info(p, "__metadata__")[0] == NH.TENSOR_NOT_FOUND


def test_files_written_by_the_safetensors_package(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(0)
    tensors = {"a.codes": rng.integers(-127, 128, size=(48, 80), dtype=np.int8),
               "a.scales": rng.random(48).astype(np.float32), "z": np.arange(5, dtype=np.uint8)}
    p = tmp_path / "pkg.safetensors"
    save_file(tensors, str(p), metadata={"format": "np"})
    raw = open(p, "rb").read()
    for name, arr in tensors.items():
        st, _, ti = info(p, name)
        assert st == NH.OK and list(ti.shape[:ti.ndim]) == list(arr.shape)
        assert ti.dtype == {np.int8: b"I8", np.float32: b"F32", np.uint8: b"U8"}[arr.dtype.type]
        assert raw[ti.data_begin:ti.data_begin + ti.data_bytes] == arr.tobytes()


def test_load_linear_validation_before_the_device(tmp_path):
    from safetensors.numpy import save_file
    p = tmp_path / "lin.safetensors"
    save_file({"w": np.zeros((32, 64), np.int8), "s": np.ones(32, np.float32), "f": np.zeros((32, 64), np.float32)},
              str(p))
    tb = NH.lib().nh_tiled_weights_bytes(32, 64)

    def load(codes, scales, n, k, staging, tiled):
        return NH.call_status("nh_load_linear_i8", None, str(p).encode(), codes.encode(), scales.encode(), n, k, 16,
                              staging, 16, tiled, 16)
    assert load("f", "s", 32, 64, 2048, tb)[0] == NH.INVALID_SHAPE  # codes must be I8
    assert load("w", "s", 32, 32, 2048, tb)[0] == NH.INVALID_SHAPE  # shape mismatch
    assert load("w", "w", 32, 64, 2048, tb)[0] == NH.INVALID_SHAPE  # scales must be F32 [n]
    st, err = load("w", "s", 32, 64, 2047, tb)
    assert st == NH.LENGTH_MISMATCH and err.argument.decode() == "staging"
    st, err = load("w", "s", 32, 64, 2048, tb - 1)
    assert st == NH.LENGTH_MISMATCH and err.argument.decode() == "tiled"
    assert load("w", "missing", 32, 64, 2048, tb)[0] == NH.TENSOR_NOT_FOUND


# ---- device ----------------------------------------------------------------
@pytest.fixture(scope="module")
def ctx():
    c = NH.Context(0)
    yield c
    c.close()


@pytest.mark.gpu
def test_read_tensor_into_device_memory(ctx, tmp_path):
    from safetensors.numpy import save_file
    x = np.random.default_rng(1).standard_normal((300, 7)).astype(np.float32)
    p = tmp_path / "x.safetensors"
    save_file({"x": x, "pad": np.zeros(3, np.uint8)}, str(p))
    d = ctx.empty(x.shape, np.float32)
    NH.call("nh_safetensors_read", ctx.handle, str(p).encode(), b"x", d.ptr, x.nbytes)
    assert np.array_equal(d.numpy(), x)
    st, err = NH.call_status("nh_safetensors_read", ctx.handle, str(p).encode(), b"x", d.ptr, x.nbytes - 4)
    assert st == NH.LENGTH_MISMATCH and err.argument.decode() == "dst"


@pytest.mark.gpu
@pytest.mark.parametrize("n,k", [(4096, 4096), (100, 1040)])
def test_load_linear_i8_then_project(ctx, tmp_path, n, k):
    from safetensors.numpy import save_file
    print(f"[gpu-case] load_linear_i8 n={n} k={k}", flush=True)
    w = O.normal_f32(0, n * k, 0.0, 0.02).reshape(n, k)
    _, q, s, _ = O.quantize_rows_f32(w)
    p = tmp_path / "layer.safetensors"
    save_file({"mixer.in_proj.codes": q, "mixer.in_proj.scales": s}, str(p))
    staging = ctx.empty(n * k, np.int8)
    tb = NH.lib().nh_tiled_weights_bytes(n, k)
    tiled = ctx.empty(tb, np.int8)
    scales = ctx.empty(n, np.float32)
    NH.call("nh_load_linear_i8", ctx.handle, str(p).encode(), b"mixer.in_proj.codes", b"mixer.in_proj.scales", n, k,
            staging.ptr, n * k, tiled.ptr, tb, scales.ptr)
    assert np.array_equal(tiled.numpy(), tile_16x64(q).reshape(-1))
    assert np.array_equal(scales.numpy().view(np.uint32), s.view(np.uint32))
    # and the layer projects exactly as the oracle does
    x = O.to_bf16(O.normal_f32(1, k)).reshape(1, k)
    _, xq, sx, _ = O.quantize_rows_bf16(x)
    dx, out = ctx.upload(x), ctx.empty((1, n), np.uint16)
    NH.call("nh_linear_w8a8", ctx.handle, dx.ptr, NH.BF16, tiled.ptr, scales.ptr, None, 1, n, k, out.ptr, NH.BF16,
            None, 0, None, None, None, None)
    ctx.synchronize()
    assert np.array_equal(out.numpy(), O.linear_w8a8(xq, sx, q, s, out_bf16=True))
