"""Checkpoint input on the host: the safetensors reader, its JSON header parser, the fp32 -> bf16
conversion and the DiT weight table's checks (everything that runs before a device is touched).

Files are written with the `safetensors` package (the format's own implementation) or byte by
byte for the malformed cases. The reference's expectations followed: src/core/safetensors.cpp
(header checks, dtypes, near-miss errors), tests/test_tensor.cpp:13-22 and 47-57 (bf16 rounding
and the JSON parser's known answers), src/core/tensor.cpp:130-160 (conversion),
src/models/weights.cpp:26-69, 246-282 (components, names and shapes)."""
from __future__ import annotations

import ctypes
import json
import struct

import numpy as np
import pytest
from safetensors.numpy import save_file

import burnisher_amd as bh
from burnisher_amd.workload import PIXART_SIGMA, block_shapes, config_struct, top_shapes, TOP_NAMES, BLOCK_NAMES
from helpers import from_bf16, to_bf16


def raw_file(path, header, data: bytes = b"", header_len=None):
    """A shard written byte by byte: u64 header length, header text, data."""
    text = header if isinstance(header, bytes) else json.dumps(header).encode()
    n = len(text) if header_len is None else header_len
    path.write_bytes(struct.pack("<Q", n) + text + data)
    return path


def open_err(*paths) -> str:
    with pytest.raises(bh.BurnisherError) as e:
        bh.Checkpoint.open(*paths)
    return str(e.value)


# ---- the header -----------------------------------------------------------------------------

def test_entries_match_what_the_format_library_wrote(tmp_path):
    rng = np.random.default_rng(1)
    tensors = {"w.weight": rng.standard_normal((3, 5)).astype(np.float32),
               "a.bias": rng.standard_normal(7).astype(np.float32),
               "h": rng.standard_normal((2, 2, 2)).astype(np.float16),
               "s": np.zeros((0, 4), np.float32)}
    p = tmp_path / "m.safetensors"
    save_file(tensors, str(p), metadata={"format": "pt"})
    with bh.Checkpoint.open(p) as ck:
        ents = ck.entries()
        assert [e[0] for e in ents] == sorted(tensors)          # name order
        got = {n: (dt, shape) for n, dt, shape in ents}
        assert got["w.weight"] == ("F32", (3, 5))
        assert got["h"] == ("F16", (2, 2, 2))
        assert got["s"] == ("F32", (0, 4))
        assert ck.has("a.bias") and not ck.has("a")
        np.testing.assert_array_equal(ck.read("w.weight", bh.F32), tensors["w.weight"])
        assert ck.read("s", bh.BF16).shape == (0, 4)


def test_json_known_answers_from_the_reference(tmp_path):
    # tests/test_tensor.cpp:48-56: this document parses; a value after the top level and an
    # empty value do not. In a header, the document sits in __metadata__, which is skipped.
    doc = b'{"a":[1,2,3],"b":{"c":"x\\ny"},"d":-1.5e2,"e":true,"f":null}'
    body = b'{"__metadata__":' + doc + b',"t":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}'
    with bh.Checkpoint.open(raw_file(tmp_path / "ok.safetensors", body, b"\0\0\x80\x3f")) as ck:
        assert ck.read("t", bh.F32).tolist() == [1.0]
    for bad in (b'{"a":1}trailing', b'{"a":}', b'{"a":[1,2}', b'{"a" 1}', b'{"a":"x', b'{"a":tru}',
                b'{"a":01x}', b'{"a":-}', b'{"a":"\\q"}', b"{'a':1}"):
        msg = open_err(raw_file(tmp_path / "bad.safetensors", bad))
        assert "json" in msg, (bad, msg)


def test_escaped_names_are_decoded(tmp_path):
    # \n, é (2-byte UTF-8), € (3-byte), a surrogate pair (4-byte) and \/
    name_json = '"x\\ny\\u00e9\\u20ac\\ud83d\\ude00\\/z"'
    body = ('{' + name_json + ':{"dtype":"BF16","shape":[2],"data_offsets":[0,4]}}').encode()
    with bh.Checkpoint.open(raw_file(tmp_path / "n.safetensors", body, b"\x80\x3f\x00\x40")) as ck:
        (name, dt, shape), = ck.entries()
        assert name == "x\nyé€😀/z" and dt == "BF16" and shape == (2,)
        assert from_bf16(ck.read(name)).tolist() == [1.0, 2.0]


def test_malformed_shards_are_refused(tmp_path):
    p = tmp_path / "x.safetensors"
    p.write_bytes(b"\x01\x00")
    assert "shorter" in open_err(p)
    assert "does not fit" in open_err(raw_file(p, b"{}", header_len=1 << 40))
    assert "does not fit" in open_err(raw_file(p, b"{}", header_len=0))
    assert "not a JSON object" in open_err(raw_file(p, b"[1,2]"))
    t = lambda **kw: {"t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8], **kw}}
    msg = open_err(raw_file(p, t(dtype="I64"), b"\0" * 16))
    assert "I64" in msg and "does not read" in msg
    assert "need 8" in open_err(raw_file(p, t(data_offsets=[0, 6]), b"\0" * 8))
    assert "need 8" in open_err(raw_file(p, t(data_offsets=[8, 0]), b"\0" * 8))
    assert "past the end" in open_err(raw_file(p, t(data_offsets=[4, 12]), b"\0" * 8))
    assert "two data_offsets" in open_err(raw_file(p, t(data_offsets=[0, 8, 8]), b"\0" * 8))
    assert "non-negative integer" in open_err(raw_file(p, t(shape=[2.5]), b"\0" * 8))
    assert "no valid 'dtype'" in open_err(raw_file(p, {"t": {"shape": [1], "data_offsets": [0, 4]}}))
    assert "cannot open" in open_err(tmp_path / "missing.safetensors")


def test_missing_names_report_near_misses(tmp_path):
    a = tmp_path / "a.safetensors"
    b = tmp_path / "b.safetensors"
    save_file({f"transformer_blocks.{i}.attn1.to_q.weight": np.zeros(2, np.float32) for i in range(7)}, str(a))
    save_file({"proj_out.bias": np.ones(2, np.float32)}, str(b))
    with bh.Checkpoint.open(a, b) as ck:
        assert ck.require("proj_out.bias") == ("F32", (2,))     # found in the second shard
        with pytest.raises(bh.BurnisherError) as e:
            ck.require("attn1.to_q.weight")
        msg = str(e.value)
        assert "missing" in msg and "Did you mean" in msg
        assert msg.count("transformer_blocks.") == 5            # at most five, name order
        assert "transformer_blocks.0.attn1" in msg and "transformer_blocks.5." not in msg
        with pytest.raises(bh.BurnisherError) as e:
            ck.require("vae.decoder.conv_in.weight")
        assert "Did you mean" not in str(e.value)


def test_component_directory(tmp_path):
    with pytest.raises(bh.BurnisherError, match="no directory"):
        bh.Checkpoint.component(tmp_path, "transformer")
    (tmp_path / "transformer").mkdir()
    (tmp_path / "transformer" / "notes.txt").write_text("x")
    with pytest.raises(bh.BurnisherError, match="no .safetensors"):
        bh.Checkpoint.component(tmp_path, "transformer")
    save_file({"b": np.ones(1, np.float32)}, str(tmp_path / "transformer" / "m-00002.safetensors"))
    save_file({"a": np.ones(1, np.float32)}, str(tmp_path / "transformer" / "m-00001.safetensors"))
    with bh.Checkpoint.component(tmp_path, "transformer") as ck:
        assert [e[0] for e in ck.entries()] == ["a", "b"]        # shards in sorted file order


# ---- conversion -------------------------------------------------------------------------------

def test_fp32_to_bf16_rounds_to_nearest_even(tmp_path):
    # tests/test_tensor.cpp:13-22 plus the cases a truncating or NaN-losing conversion fails
    vals = np.array([1.0, 0.0, -2.5, 1.0 + 2.0 ** -9, 1.0 + 3 * 2.0 ** -9, -0.0, np.inf, -np.inf,
                     np.nan, 1e-40, -1e-45, 3.4028235e38, 1.0 + 2.0 ** -8 + 2.0 ** -20], np.float32)
    rng = np.random.default_rng(2)
    big = (rng.standard_normal(3_000_001) * 10.0 ** rng.integers(-30, 30, 3_000_001)).astype(np.float32)
    p = tmp_path / "c.safetensors"
    save_file({"v": vals, "big": big}, str(p))
    with bh.Checkpoint.open(p) as ck:
        got = ck.read("v", bh.BF16)
        f = from_bf16(got)
        assert f[0] == 1.0 and f[1] == 0.0 and f[2] == -2.5
        assert f[3] == 1.0                                      # the tie goes to even
        assert f[4] == 1.0 + 2.0 ** -7                          # above the tie rounds up
        assert got[5] == 0x8000 and np.isinf(f[6]) and np.isinf(f[7]) and np.isnan(f[8])
        assert f[12] == 1.0 + 2.0 ** -7
        np.testing.assert_array_equal(got, to_bf16(vals))
        # multi-threaded path: bytes do not depend on the split
        np.testing.assert_array_equal(ck.read("big", bh.BF16), to_bf16(big))
    # bf16 stored as BF16 is copied exactly and widens exactly
    bits = to_bf16(big[:1000])
    raw = bits.tobytes()
    q = raw_file(tmp_path / "bf.safetensors",
                 {"b": {"dtype": "BF16", "shape": [1000], "data_offsets": [0, len(raw)]}}, raw)
    with bh.Checkpoint.open(q) as ck:
        np.testing.assert_array_equal(ck.read("b", bh.BF16), bits)
        np.testing.assert_array_equal(ck.read("b", bh.F32), from_bf16(bits))


def test_f16_and_fp8_are_named_but_not_converted(tmp_path):
    # recognised at open (safetensors.cpp:186-195), refused at conversion (tensor.cpp:68-82)
    body = {"h": {"dtype": "F16", "shape": [2], "data_offsets": [0, 4]},
            "e": {"dtype": "F8_E4M3", "shape": [4], "data_offsets": [4, 8]}}
    with bh.Checkpoint.open(raw_file(tmp_path / "h.safetensors", body, b"\0" * 8)) as ck:
        assert {n: dt for n, dt, _ in ck.entries()} == {"h": "F16", "e": "F8_E4M3"}
        for name in ("h", "e"):
            with pytest.raises(bh.BurnisherError, match="no per-element conversion"):
                ck.read(name)


def test_read_checks_the_element_count(tmp_path):
    p = tmp_path / "r.safetensors"
    save_file({"t": np.ones(6, np.float32)}, str(p))
    with bh.Checkpoint.open(p) as ck:
        out = np.zeros(5, np.uint16)
        with pytest.raises(bh.BurnisherError, match="6 elements"):
            bh.call("bh_checkpoint_read", ck.handle, b"t", bh.BF16, out.ctypes.data, 5)


# ---- the DiT's weight table (checked before any device allocation) ----------------------------

def dit_tensors(cfg: dict) -> dict[str, tuple]:
    out = {TOP_NAMES[k]: s for k, s in top_shapes(cfg).items()}
    for i in range(cfg["num_layers"]):
        for k, s in block_shapes(cfg).items():
            out[f"transformer_blocks.{i}.{BLOCK_NAMES[k]}"] = s
    return out


def tiny_cfg(layers=2) -> dict:
    return dict(PIXART_SIGMA, num_layers=layers, num_heads=2, head_dim=8, caption_channels=24)


def write_dit(path, cfg, *, drop=None, reshape=None, dtype=np.float32):
    tensors = {n: np.zeros(s, dtype) for n, s in dit_tensors(cfg).items()}
    if drop:
        del tensors[drop]
    if reshape:
        tensors[reshape[0]] = np.zeros(reshape[1], dtype)
    save_file(tensors, str(path))
    return path


def load_err(path, cfg) -> str:
    with bh.Checkpoint.open(path) as ck, pytest.raises(bh.BurnisherError) as e:
        bh.DitDeviceWeights(ck, config_struct(cfg))
    return str(e.value)


def test_dit_table_matches_the_published_layout():
    # configs/checkpoint-layout.json of the reference lists the pinned checkpoint's tensors;
    # the DiT's 603 of them are these names and shapes at the PixArt-Sigma configuration
    names = dit_tensors(PIXART_SIGMA)
    assert len(names) == 15 + 28 * 21 == 603
    assert names["pos_embed.proj.weight"] == (1152, 4, 2, 2)
    assert names["adaln_single.linear.weight"] == (6912, 1152)
    assert names["caption_projection.linear_1.weight"] == (1152, 4096)
    assert names["proj_out.weight"] == (32, 1152)
    assert names["transformer_blocks.27.ff.net.0.proj.weight"] == (4608, 1152)
    assert names["transformer_blocks.0.scale_shift_table"] == (6, 1152)


def test_dit_load_refuses_before_allocating(tmp_path):
    cfg = tiny_cfg()
    p = write_dit(tmp_path / "drop.safetensors", cfg, drop="transformer_blocks.1.attn2.to_k.bias")
    msg = load_err(p, cfg)
    assert "'transformer_blocks.1.attn2.to_k.bias' is missing" in msg and "fatal" in msg
    p = write_dit(tmp_path / "shape.safetensors", cfg, reshape=("transformer_blocks.0.ff.net.2.weight", (16, 32)))
    msg = load_err(p, cfg)
    assert "[16, 32] in the checkpoint" in msg and "needs [16, 64]" in msg
    p = write_dit(tmp_path / "f16.safetensors", cfg, dtype=np.float16)
    assert "no per-element conversion" in load_err(p, cfg)
    # more layers than the checkpoint holds
    p = write_dit(tmp_path / "ok.safetensors", cfg)
    assert "transformer_blocks.2." in load_err(p, tiny_cfg(layers=3))
