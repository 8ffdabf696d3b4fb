"""The C ABI (include/qe.h) without a GPU: every declared symbol is exported by libqe.so, and the
loader's contract violations come back as status codes (the reference panics on them:
cpu_inference.rs:62-96, metal_inference.rs:247)."""
import ctypes
import json
import os
import re
import struct

import pytest

import qe

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TINY = qe.Config(256, 512, 2, 4, 2, 128, 1000, 1e-6, 1e6, 999)


def declared_functions():
    text = open(os.path.join(ROOT, "include", "qe.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qe_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert len(names) >= 18
    lib = ctypes.CDLL(qe.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def gpu_visible():
    try:
        import torch

        return torch.cuda.is_available()
    except ImportError:
        return False


def load_err(path):
    with pytest.raises(qe.QeError) as e:
        qe.Model.load_model(path)
    return e.value.code, str(e.value)


def write_st(path, header: dict, data: bytes, pad_to=8, config=True):
    h = json.dumps(header).encode()
    while pad_to and (8 + len(h)) % pad_to:
        h += b" "
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + data)
    if config:
        cfg = {"hidden_size": 256, "intermediate_size": 512, "num_hidden_layers": 2, "num_attention_heads": 4,
               "num_key_value_heads": 2, "head_dim": 128, "vocab_size": 1000, "rms_norm_eps": 1e-6,
               "rope_theta": 1000000.0, "eos_token_id": 999}
        with open(os.path.join(os.path.dirname(path), "config.json"), "w") as f:
            json.dump(cfg, f)


def test_missing_file(tmp_path):
    code, _ = load_err(str(tmp_path / "nope.safetensors"))
    assert code == qe.QE_ERR_IO


def test_truncated_and_garbled_headers(tmp_path):
    p = tmp_path / "m.safetensors"
    p.write_bytes(b"\x01\x02\x03")
    assert load_err(str(p))[0] == qe.QE_ERR_FORMAT
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    assert load_err(str(p))[0] == qe.QE_ERR_FORMAT
    p.write_bytes(struct.pack("<Q", 5) + b"{nope")
    assert load_err(str(p))[0] == qe.QE_ERR_FORMAT


def test_misaligned_data_section(tmp_path):
    p = str(tmp_path / "m.safetensors")
    write_st(p, {"x": {"dtype": "BF16", "shape": [1], "data_offsets": [0, 2]}}, b"\0\0", pad_to=0)
    hl = int.from_bytes(open(p, "rb").read(8), "little")
    if (8 + hl) % 2 == 0:  # make the header odd-length so the data starts at an odd offset
        write_st(p, {"xx": {"dtype": "BF16", "shape": [1], "data_offsets": [0, 2]}}, b"\0\0", pad_to=0)
    assert (8 + int.from_bytes(open(p, "rb").read(8), "little")) % 2 == 1
    code, msg = load_err(p)
    assert code == qe.QE_ERR_FORMAT and "aligned" in msg


def test_missing_config(tmp_path):
    p = str(tmp_path / "m.safetensors")
    write_st(p, {"__metadata__": {"format": "pt"}}, b"", config=False)
    assert load_err(p)[0] == qe.QE_ERR_IO


def test_config_missing_field(tmp_path):
    p = str(tmp_path / "m.safetensors")
    write_st(p, {}, b"")
    cfg = json.load(open(tmp_path / "config.json"))
    del cfg["rope_theta"]
    json.dump(cfg, open(tmp_path / "config.json", "w"))
    assert load_err(p)[0] == qe.QE_ERR_FORMAT


def test_missing_tensor_wrong_dtype_wrong_shape(tmp_path):
    path = qe.write_random_checkpoint(str(tmp_path / "ok"), 1, TINY)
    raw = open(path, "rb").read()
    hl = int.from_bytes(raw[:8], "little")
    header = json.loads(raw[8:8 + hl])
    data = raw[8 + hl:]
    cases = {}
    h1 = dict(header)
    del h1["model.layers.1.mlp.down_proj.weight"]
    cases["missing"] = h1
    h2 = json.loads(json.dumps(header))
    h2["model.layers.0.self_attn.k_norm.weight"]["dtype"] = "F16"
    cases["dtype"] = h2
    h3 = json.loads(json.dumps(header))
    h3["model.layers.0.self_attn.q_norm.weight"]["shape"] = [64]
    cases["shape"] = h3
    # an odd data offset: the reference views the bytes in place as u16 (cpu_inference.rs:95)
    h4 = json.loads(json.dumps(header))
    t = h4["model.layers.0.self_attn.q_norm.weight"]
    t["data_offsets"] = [t["data_offsets"][0] + 1, t["data_offsets"][1] + 1]
    cases["odd_offset"] = h4
    for name, h in cases.items():
        d = tmp_path / name
        d.mkdir()
        p = str(d / "model.safetensors")
        write_st(p, h, data)
        code, msg = load_err(p)
        assert code == qe.QE_ERR_TENSOR, (name, msg)


def test_bad_offsets_and_overflowing_shapes(tmp_path):
    """an entry the engine never loads still needs a byte range inside the data section (the byte
    formula sums every entry's off1 - off0), and a shape whose element count wraps around 2^64 to
    the expected count is rejected rather than accepted"""
    path = qe.write_random_checkpoint(str(tmp_path / "ok"), 1, TINY)
    raw = open(path, "rb").read()
    hl = int.from_bytes(raw[:8], "little")
    header = json.loads(raw[8:8 + hl])
    data = raw[8 + hl:]
    cases = {}
    for name, offs in {"reversed": [10, 4], "negative": [-2, 4], "past_end": [0, len(data) + 2]}.items():
        h = json.loads(json.dumps(header))
        h["extra.unused"] = {"dtype": "BF16", "shape": [2], "data_offsets": offs}
        cases[name] = (h, qe.QE_ERR_FORMAT)
    # q_norm has 128 elements: 99789673 * 1444189401 = 2^57 + 1, so with a dim of 128 the product
    # is 2^64 + 128, which wraps to 128 in 64-bit arithmetic (every dim fits an i32)
    h = json.loads(json.dumps(header))
    assert 99789673 * 1444189401 == 2 ** 57 + 1
    h["model.layers.0.self_attn.q_norm.weight"]["shape"] = [99789673, 1444189401, 128]
    cases["wrapping_shape"] = (h, qe.QE_ERR_TENSOR)
    for name, (h, want) in cases.items():
        d = tmp_path / name
        d.mkdir()
        p = str(d / "model.safetensors")
        write_st(p, h, data)
        code, msg = load_err(p)
        assert code == want, (name, msg)


@pytest.mark.skipif(gpu_visible(), reason="with a GPU the valid file loads; covered by the gpu tests")
def test_valid_file_reports_no_device(tmp_path):
    path = qe.write_random_checkpoint(str(tmp_path), 1, TINY)
    code, msg = load_err(path)
    assert code == qe.QE_ERR_NO_DEVICE


def test_null_arguments():
    L = qe.lib()
    assert L.qe_model_load(None, None) == qe.QE_ERR_ARG
    assert b"null" in L.qe_last_error()
    assert L.qe_kv_new(None, 16, 0, None) == qe.QE_ERR_ARG
    assert L.qe_forward(None, 0, 0, None, None) == qe.QE_ERR_ARG
