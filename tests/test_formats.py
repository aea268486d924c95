"""On-disk formats on the CPU: the local safetensors reader against files
written two independent ways -- by hand from the format's definition (8-byte
little-endian header length, JSON header, raw little-endian tensors; the
reference's own test writes its fake checkpoint this way,
tests/test_gpt2.py:25-38) and by the ``safetensors`` package -- and the
checkpoint lookups' behaviour when no checkpoint is present."""

import json
import struct

import numpy as np
import pytest

from draftkv.gpt2 import load_safetensors


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def _write(path, tensors: dict) -> None:
    """tensors: name -> (dtype tag, raw little-endian bytes, shape)."""
    header, blobs, off = {"__metadata__": {"format": "pt"}}, [], 0
    for name, (tag, raw, shape) in tensors.items():
        header[name] = {"dtype": tag, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)                         # writers pad the header to 8 bytes
    path.write_bytes(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def test_roundtrip_f32_bf16_f16_hand_written(tmp_path):
    rng = np.random.default_rng(0)
    a = rng.standard_normal((3, 4)).astype(np.float32)
    b = rng.standard_normal(7).astype(np.float32)
    c = rng.standard_normal((2, 3, 4)).astype(np.float32)
    bits = _bf16_bits(c)
    d = rng.standard_normal((5, 2)).astype(np.float16)
    e = np.arange(-3, 3, dtype=np.int64)
    f = tmp_path / "model.safetensors"
    _write(f, {"a": ("F32", a.tobytes(), a.shape), "b": ("F32", b.tobytes(), b.shape),
               "c.nested.weight": ("BF16", bits.tobytes(), c.shape), "d": ("F16", d.tobytes(), d.shape),
               "e": ("I64", e.tobytes(), e.shape), "scalar": ("F32", np.float32(2.5).tobytes(), ())})
    got = load_safetensors(f)
    assert set(got) == {"a", "b", "c.nested.weight", "d", "e", "scalar"}
    assert all(v.dtype == np.float32 for v in got.values())
    assert np.array_equal(got["a"], a) and np.array_equal(got["b"], b)
    # bf16 widens exactly: the loaded float32 holds the stored bits in its top half
    want_c = (bits.astype(np.uint32) << 16).view(np.float32)
    assert got["c.nested.weight"].shape == (2, 3, 4)
    assert np.array_equal(got["c.nested.weight"].view(np.uint32), want_c.view(np.uint32))
    assert np.abs(got["c.nested.weight"] - c).max() <= np.abs(c).max() * 2.0 ** -8
    assert np.array_equal(got["d"], d.astype(np.float32))
    assert np.array_equal(got["e"], e.astype(np.float32))
    assert got["scalar"].shape == () and float(got["scalar"]) == 2.5


def test_roundtrip_against_the_safetensors_package(tmp_path):
    st = pytest.importorskip("safetensors.numpy")
    rng = np.random.default_rng(1)
    arrays = {"wte.weight": rng.standard_normal((11, 8)).astype(np.float32),
              "h.0.attn.c_attn.weight": rng.standard_normal((8, 24)).astype(np.float32),
              "h.0.ln_1.bias": np.zeros(8, np.float32), "half": rng.standard_normal(6).astype(np.float16)}
    f = tmp_path / "m.safetensors"
    st.save_file(arrays, str(f))
    got = load_safetensors(f)
    assert set(got) == set(arrays)
    for k, v in arrays.items():
        assert np.array_equal(got[k], v.astype(np.float32)), k


def test_unsupported_dtype_is_refused(tmp_path):
    f = tmp_path / "bad.safetensors"
    _write(f, {"x": ("F8_E4M3", b"\x00" * 4, (4,))})
    with pytest.raises(ValueError, match="unsupported dtype"):
        load_safetensors(f)


def test_missing_checkpoints_raise_file_not_found(tmp_path, monkeypatch):
    from draftkv import gpt2, llama
    monkeypatch.setenv("DRAFTKV_GPT2_DIR", str(tmp_path / "none"))
    monkeypatch.setenv("HOME", str(tmp_path))
    if gpt2.default_model_dir() is None:
        with pytest.raises(FileNotFoundError):
            gpt2.load_real_model()
    with pytest.raises(FileNotFoundError):
        llama.load_llama(tmp_path / "absent")
