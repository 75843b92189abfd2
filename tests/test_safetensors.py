"""The safetensors reader (the reference's safetensors::Files, tests/safetensors_test.cpp:36-98) through the C ABI, on
the host only: files written by the `safetensors` package (an independent writer of the format), sharded directories,
dims in GGUF order (dims[0] contiguous), absolute data offsets, and every malformed header turned into an error."""
import json
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import mkimage


def tensors():
    g = torch.Generator().manual_seed(0)
    return {
        "img_in.weight": torch.randn(3, 5, generator=g).to(torch.bfloat16),
        "b.vec": torch.randn(7, generator=g),
        "c.half": torch.randn(2, 3, 4, generator=g).to(torch.float16),
        "d.fp8": (torch.randn(4, 2, generator=g) * 8).to(torch.float8_e4m3fn),
        "e.int": torch.arange(3, dtype=torch.int64),
        "f.empty": torch.zeros(0, 4),
        "g.scalar": torch.tensor(2.5),
    }


def raw(t):
    return t.contiguous().reshape(-1).view(torch.uint8).numpy().tobytes() if t.numel() else b""


def test_reads_what_the_safetensors_package_wrote(tmp_path):
    ts = tensors()
    path = tmp_path / "m.safetensors"
    save_file(ts, str(path), metadata={"format": "pt"})
    st = mkimage.SafeTensors(path)
    assert len(st) == len(ts)
    assert st.files() == [str(path)]
    codes = {torch.bfloat16: mkimage.BF16, torch.float32: mkimage.F32, torch.float16: mkimage.F16,
             torch.float8_e4m3fn: mkimage.FP8, torch.int64: mkimage.DTYPE_OTHER}
    names = {"F8_E4M3", "BF16", "F32", "F16", "I64"}
    data = path.read_bytes()
    for name, t in ts.items():
        info = st.find(name)
        assert info["dims"] == list(reversed(t.shape)), name  # GGUF order
        assert info["dtype"] == codes[t.dtype], name
        assert info["dtype_name"] in names
        assert info["bytes"] == t.numel() * t.element_size()
        want = raw(t)
        assert st.read(name).tobytes() == want, name
        # the offset is absolute in the file (the reference reads the first values at it)
        assert data[info["offset"]:info["offset"] + info["bytes"]] == want, name
    # the reference test's check: the first bf16 values of a matrix at its offset, as the file's own reader gives
    info = st.find("img_in.weight")
    first = np.frombuffer(data[info["offset"]:info["offset"] + 8], dtype=np.uint16)
    assert np.array_equal(mkimage.bf16_to_f32(first), ts["img_in.weight"].float().flatten()[:4].numpy())
    assert {t["name"] for t in st.tensors()} == set(ts)


def test_shard_directory(tmp_path):
    ts = tensors()
    keys = sorted(ts)
    save_file({k: ts[k] for k in keys[:3]}, str(tmp_path / "model-00002-of-00002.safetensors"))
    save_file({k: ts[k] for k in keys[3:]}, str(tmp_path / "model-00001-of-00002.safetensors"))
    (tmp_path / "model.safetensors.index.json").write_text("{}")
    st = mkimage.SafeTensors(tmp_path)
    files = st.files()
    assert [f.rsplit("/", 1)[1] for f in files] == ["model-00001-of-00002.safetensors",
                                                     "model-00002-of-00002.safetensors"]
    assert len(st) == len(ts)
    for name, t in ts.items():
        info = st.find(name)
        assert files[info["file"]].endswith("00001-of-00002.safetensors") == (name in keys[3:])
        assert st.read(name).tobytes() == raw(t)
    # the same name in two shards is an error
    save_file({keys[0]: ts[keys[0]]}, str(tmp_path / "model-00003.safetensors"))
    with pytest.raises(mkimage.MkError, match="twice"):
        mkimage.SafeTensors(tmp_path)


def write(path, header, data=b"", pad=True):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    if pad:
        h += b" " * (-len(h) % 8)
    path.write_bytes(struct.pack("<Q", len(h)) + h + data)
    return path


def test_hand_written_header_escapes_and_metadata(tmp_path):
    hdr = ('{"__metadata__": {"k": "v \\"q\\"", "n": {"x": [1, 2.5e3, true, null]}}, '
           '"caf\\u00e9.\\"w\\"": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}, '
           '"z": {"data_offsets": [8, 10], "shape": [1], "dtype": "BF16"}}').encode()
    data = np.array([1.0, -2.0], np.float32).tobytes() + b"\x80\x3f"
    st = mkimage.SafeTensors(write(tmp_path / "e.safetensors", hdr, data))
    assert sorted(t["name"] for t in st.tensors()) == ['café."w"', "z"]
    assert np.array_equal(np.frombuffer(st.read('café."w"').tobytes(), np.float32), [1.0, -2.0])
    assert st.find("z")["offset"] == 8 + len(hdr) + (-len(hdr) % 8) + 8
    with pytest.raises(mkimage.MkError, match="no tensor named"):
        st.find("absent")


@pytest.mark.parametrize("case, match", [
    ("short", "shorter"),
    ("huge_header", "does not fit"),
    ("not_json", "not a JSON object"),
    ("bad_size", "bytes for"),
    ("beyond", "outside"),
    ("dtype", "unknown dtype"),
    ("missing_key", "lacks"),
    ("reversed", "outside"),
    ("trailing", "trailing"),
    ("float_shape", "integer"),
    ("unterminated", "bad header entry"),
])
def test_malformed_files_are_errors(tmp_path, case, match):
    p = tmp_path / f"{case}.safetensors"
    ok = {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}
    data = bytes(8)
    if case == "short":
        p.write_bytes(b"\x01\x02")
    elif case == "huge_header":
        p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    elif case == "not_json":
        write(p, b"[1, 2]", data)
    elif case == "bad_size":
        write(p, {"a": {**ok, "shape": [3]}}, data)
    elif case == "beyond":
        write(p, {"a": {**ok, "data_offsets": [0, 16]}}, data)
    elif case == "dtype":
        write(p, {"a": {**ok, "dtype": "Q4"}}, data)
    elif case == "missing_key":
        write(p, {"a": {"dtype": "F32", "shape": [2]}}, data)
    elif case == "reversed":
        write(p, {"a": {**ok, "data_offsets": [8, 0]}}, data)
    elif case == "trailing":
        write(p, json.dumps({"a": ok}).encode() + b" x", data, pad=False)
    elif case == "float_shape":
        write(p, b'{"a": {"dtype": "F32", "shape": [2.0], "data_offsets": [0, 8]}}', data)
    elif case == "unterminated":
        write(p, b'{"a', data)
    with pytest.raises(mkimage.MkError, match=match):
        mkimage.SafeTensors(p)


def test_missing_paths_and_empty_directory(tmp_path):
    with pytest.raises(mkimage.MkError, match="no such file"):
        mkimage.SafeTensors(tmp_path / "nope.safetensors")
    with pytest.raises(mkimage.MkError, match="no \\*.safetensors"):
        mkimage.SafeTensors(tmp_path)
