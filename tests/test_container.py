"""The `.fni8` container and loader (fni8serve_amd.container, fni8serve_amd.loader).

Mirrors the reference's own container tests: the save -> load round trip and
the LinearW8A8 seam on the loaded weights (tests/test_smoke.py:32-49), partial
loads through the shard index (test_smoke.py:58-64), the byte-exact round trip
(tests/test_convert.py:120-136) and checkpoint_info's header fields
(test_convert.py:359-362).  The reference's byte layout lives in its closed
`fni8.format` and is not restated: what is pinned here is this container's own
layout (aligned blobs in resident layout, the trailer, version checks) and that
every loaded tensor is bitwise the one saved.
"""
import json
import os
import struct

import pytest
import torch

from fni8serve_amd import LinearW8A8, QTensor, quantize_int8_rowwise
from fni8serve_amd.container import ALIGN, ARCH, FORMAT_VERSION, MAGIC, FQReader, FQWriter, save_fni8
from fni8serve_amd.loader import checkpoint_info, load_fni8_checkpoint, load_fni8_state_dict


def _i8(out, in_, seed=0):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(out, in_, generator=g)
    q, s = quantize_int8_rowwise(w)
    return QTensor(q, s.squeeze(-1), scheme="per_row_i8")


def _i4(out, in_, gs, seed=0):
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(-7, 8, (out, in_), generator=g)
    u = (codes & 0xF).to(torch.int32)
    packed = (u[:, 0::2] | (u[:, 1::2] << 4)).to(torch.uint8)
    scale = torch.rand(out, in_ // gs, generator=g) + 0.01
    return QTensor(packed, scale, scheme="per_group_i4", group_size=gs, codebook="int4")


def _same(a: QTensor, b: QTensor):
    assert (a.scheme, a.group_size, a.codebook) == (b.scheme, b.group_size, b.codebook)
    assert a.data.dtype == b.data.dtype and a.data.shape == b.data.shape
    assert torch.equal(a.data.view(torch.uint8) if a.data.dtype != torch.bool else a.data,
                       b.data.view(torch.uint8) if b.data.dtype != torch.bool else b.data)
    if a.scale is None:
        assert b.scale is None
    else:
        assert a.scale.dtype == b.scale.dtype and torch.equal(a.scale.view(torch.uint8),
                                                              b.scale.view(torch.uint8))


def _mixed():
    g = torch.Generator().manual_seed(3)
    return {
        "model.layers.0.mlp.gate_up_proj.weight": _i8(96, 64, 1),
        "model.layers.0.mlp.down_proj.weight": _i4(64, 128, 32, 2),
        "model.layers.0.input_layernorm.weight": torch.randn(64, generator=g).half(),
        "model.embed_tokens.weight": torch.randn(50, 64, generator=g).to(torch.bfloat16),
        "model.layers.0.mlp.gate.weight": torch.randn(8, 64, generator=g),
        "model.layers.0.router.bias": torch.empty(0, dtype=torch.float16),
        "lm_head.weight": _i8(50, 64, 4),
    }


def test_roundtrip_load_and_linear_w8(tmp_path):
    path = str(tmp_path / "m.fni8")
    qt = _i8(128, 256)
    save_fni8(path, {"mlp.up.weight": qt})
    w = load_fni8_checkpoint(path, device="cpu")
    assert list(w) == ["mlp.up.weight"]
    _same(w["mlp.up.weight"], qt)
    lin = LinearW8A8(w["mlp.up.weight"])
    y = lin(torch.randn(4, 256))
    assert y.shape == (4, 128) and torch.isfinite(y).all()


def test_linear_w4_seam(tmp_path):
    path = str(tmp_path / "m.fni8")
    save_fni8(path, {"mlp.down.weight": _i4(64, 128, 32)})
    w = load_fni8_checkpoint(path, device="cpu")
    lin = LinearW8A8(w["mlp.down.weight"])
    assert lin.in_features == 128 and lin.out_features == 64
    y = lin(torch.randn(2, 128))
    assert y.shape == (2, 64) and torch.isfinite(y).all()


def test_every_scheme_and_dtype_roundtrips_bitwise(tmp_path):
    path = str(tmp_path / "m.fni8")
    ts = _mixed()
    save_fni8(path, ts, meta={"arch": "qwen3", "hidden_size": 64})
    got = load_fni8_checkpoint(path, device="cpu")
    assert list(got) == list(ts)
    for name, obj in ts.items():
        ref = obj if isinstance(obj, QTensor) else QTensor(obj, None, scheme="raw")
        _same(got[name], ref)


def test_blobs_are_aligned_and_in_resident_layout(tmp_path):
    """Each blob starts on a 4096-byte boundary and holds the tensor's bytes as
    they sit in memory (row-major, no transform), so the file region can be
    mapped or copied straight into the kernel's operand."""
    path = str(tmp_path / "m.fni8")
    ts = _mixed()
    save_fni8(path, ts)
    raw = open(path, "rb").read()
    assert raw[:8] == MAGIC and struct.unpack_from("<I", raw, 8)[0] == FORMAT_VERSION
    with FQReader(path) as r:
        for name, t in r.header["tensors"].items():
            obj = ts[name]
            qt = obj if isinstance(obj, QTensor) else QTensor(obj, None, scheme="raw")
            for part, ten in (("data", qt.data), ("scale", qt.scale)):
                b = t[part]
                if ten is None:
                    assert b is None
                    continue
                assert b["offset"] % ALIGN == 0
                assert b["nbytes"] == ten.numel() * ten.element_size()
                mine = ten.contiguous().view(torch.uint8).reshape(-1).numpy().tobytes()
                assert raw[b["offset"]:b["offset"] + b["nbytes"]] == mine


def test_noncontiguous_input_is_stored_row_major(tmp_path):
    path = str(tmp_path / "m.fni8")
    q = _i8(64, 32).data.t()  # [32, 64] view with strides (1, 32)
    qt = QTensor(q, torch.rand(32), scheme="per_row_i8")
    save_fni8(path, {"w": qt})
    got = load_fni8_checkpoint(path, device="cpu")["w"]
    assert got.data.is_contiguous() and torch.equal(got.data, q)


def test_shard_partial_load(tmp_path):
    path = str(tmp_path / "m.fni8")
    ts = {f"model.layers.{i}.w": _i8(32, 64, i) for i in range(4)}
    save_fni8(path, ts, shards={"pp_stages": [["model.layers.0.w", "model.layers.1.w"],
                                              ["model.layers.2.w", "model.layers.3.w"]]})
    w = load_fni8_checkpoint(path, device="cpu", shard="pp:1")
    assert set(w) == {"model.layers.2.w", "model.layers.3.w"}
    _same(w["model.layers.3.w"], ts["model.layers.3.w"])
    w0 = load_fni8_checkpoint(path, device="cpu", shard="pp:0")
    assert set(w0) == {"model.layers.0.w", "model.layers.1.w"}


def test_expert_shard_and_names(tmp_path):
    path = str(tmp_path / "m.fni8")
    ts = {f"experts.{e}.{p}": _i8(16, 32, 10 * e + i)
          for e in range(3) for i, p in enumerate(("gate_up", "down"))}
    shards = {"experts": {str(e): [f"experts.{e}.gate_up", f"experts.{e}.down"] for e in range(3)}}
    save_fni8(path, ts, shards=shards)
    w = load_fni8_checkpoint(path, device="cpu", shard="2")
    assert set(w) == {"experts.2.gate_up", "experts.2.down"}
    _same(w["experts.2.down"], ts["experts.2.down"])
    w = load_fni8_checkpoint(path, device="cpu", names=["experts.0.down"])
    assert list(w) == ["experts.0.down"]
    with pytest.raises(KeyError, match="unknown shard"):
        load_fni8_checkpoint(path, device="cpu", shard="7")
    with pytest.raises(KeyError):
        load_fni8_checkpoint(path, device="cpu", shard="pp:0")  # no pp_stages in this index
    with pytest.raises(KeyError, match="no tensor"):
        load_fni8_checkpoint(path, device="cpu", names=["experts.9.down"])


def test_zero_dim_raw_tensors_roundtrip(tmp_path):
    """0-d tensors (an optimizer's step count, a scalar buffer) as the reference's
    training checkpoint writes them through save_fni8 (loader.py save_training_checkpoint)."""
    path = str(tmp_path / "m.fni8")
    ts = {"optimizer.state.0.step": torch.tensor(3.0), "count": torch.tensor(7, dtype=torch.int64),
          "half": torch.tensor(-1.5, dtype=torch.float16)}
    save_fni8(path, ts)
    sd = load_fni8_state_dict(path, device="cpu")
    for name, t in ts.items():
        assert sd[name].shape == t.shape and sd[name].dtype == t.dtype
        assert torch.equal(sd[name], t)


def test_state_dict_unwraps_raw(tmp_path):
    path = str(tmp_path / "m.fni8")
    ts = _mixed()
    save_fni8(path, ts)
    sd = load_fni8_state_dict(path, device="cpu")
    for name, obj in ts.items():
        if isinstance(obj, QTensor):
            assert isinstance(sd[name], QTensor)
        else:
            assert isinstance(sd[name], torch.Tensor) and not isinstance(sd[name], QTensor)
            assert sd[name].dtype == obj.dtype and torch.equal(sd[name], obj)


def test_checkpoint_info(tmp_path):
    path = str(tmp_path / "m.fni8")
    ts = {f"l{i}": _i8(8, 16, i) for i in range(4)}
    ts["norm"] = torch.ones(16, dtype=torch.float16)
    save_fni8(path, ts, shards={"pp_stages": [["l0", "l1"], ["l2", "l3", "norm"]],
                                "experts": {"0": ["l0"]}},
              meta={"arch": "qwen3", "num_hidden_layers": 4})
    info = checkpoint_info(path)
    # header "arch" is the hardware target; the model's arch lives in meta
    assert info == {"arch": ARCH, "quant": "per_row_i8", "version": FORMAT_VERSION,
                    "num_tensors": 5, "shards": {"pp_stages": 2, "experts": 1},
                    "meta": {"arch": "qwen3", "num_hidden_layers": 4}}
    path2 = str(tmp_path / "mixed.fni8")
    save_fni8(path2, _mixed())
    assert checkpoint_info(path2)["quant"] == "mixed"
    assert checkpoint_info(path2)["shards"] == {}


def test_streaming_writer_matches_save(tmp_path):
    """FQWriter.add one tensor at a time then finalize(meta=) -- the converter's
    pattern (fni8serve/convert.py:318-361) -- gives the same file as save_fni8."""
    ts = _mixed()
    a, b = str(tmp_path / "a.fni8"), str(tmp_path / "b.fni8")
    w = FQWriter(a)
    for name, obj in ts.items():
        w.add(name, obj)
    w.finalize(meta={"k": 1})
    save_fni8(b, ts, meta={"k": 1})
    assert open(a, "rb").read() == open(b, "rb").read()
    with FQReader(a) as r:
        assert r.names == list(ts) and r.header["__meta__"] == {"k": 1}


def test_writer_errors_and_partial_file_removed(tmp_path):
    path = str(tmp_path / "m.fni8")
    w = FQWriter(path)
    w.add("a", _i8(8, 16))
    with pytest.raises(ValueError, match="duplicate"):
        w.add("a", _i8(8, 16))
    with pytest.raises(TypeError):
        w.add("b", [1, 2, 3])
    with pytest.raises(KeyError, match="unknown tensors"):
        w.finalize(shards={"pp_stages": [["a", "missing"]]})
    w.close()
    assert not os.path.exists(path)
    with pytest.raises(RuntimeError):
        with FQWriter(path) as w2:
            w2.add("a", _i8(8, 16))
            raise RuntimeError("converter failed mid-stream")
    assert not os.path.exists(path)


@pytest.mark.parametrize("damage", ["magic", "version", "truncate", "trailer", "offset",
                                    "shape", "dtype"])
def test_reader_rejects_damaged_files(tmp_path, damage):
    path = str(tmp_path / "m.fni8")
    save_fni8(path, {"a": _i8(8, 16), "b": _i8(4, 16, 1)})
    raw = bytearray(open(path, "rb").read())
    if damage == "magic":
        raw[0:8] = b"NOTFNI8\0"
    elif damage == "version":
        raw[8:12] = struct.pack("<I", FORMAT_VERSION + 1)
    elif damage == "truncate":
        raw = raw[:len(raw) - 5]
    elif damage == "trailer":
        raw[-8:] = b"XXXXXXXX"
    else:  # the header: a blob past the data region, a shape that is not its bytes, a bad dtype
        hoff, hlen, _ = struct.unpack_from("<QQ8s", raw, len(raw) - 24)
        h = json.loads(bytes(raw[hoff:hoff + hlen]))
        d = h["tensors"]["b"]["data"]
        if damage == "offset":
            d["offset"] = hoff
        elif damage == "shape":
            d["shape"] = [5, 16]
        else:
            d["dtype"] = "complex32"
        blob = json.dumps(h, separators=(",", ":")).encode()
        raw = raw[:hoff] + blob + struct.pack("<QQ8s", hoff, len(blob), MAGIC)
    open(path, "wb").write(bytes(raw))
    with pytest.raises(ValueError):
        FQReader(path)


def test_reader_rejects_tiny_file(tmp_path):
    path = str(tmp_path / "m.fni8")
    open(path, "wb").write(MAGIC)
    with pytest.raises(ValueError, match="too short"):
        FQReader(path)


def test_empty_checkpoint(tmp_path):
    path = str(tmp_path / "m.fni8")
    save_fni8(path, {})
    assert load_fni8_checkpoint(path, device="cpu") == {}
    assert checkpoint_info(path)["num_tensors"] == 0


@pytest.mark.gpu
@pytest.mark.parametrize("chunk", [None, 12_345])
def test_device_load_is_bitwise(tmp_path, monkeypatch, chunk):
    """The device load (pinned ring + side-stream copies) gives the saved bytes,
    with a 41 MB blob split over several 32 MiB chunks, and with a tiny odd chunk
    so that every staging buffer is reused many times."""
    from fni8serve_amd import container
    if chunk is not None:
        monkeypatch.setattr(container, "_CHUNK", chunk)
    path = str(tmp_path / "m.fni8")
    ts = _mixed()
    ts["big"] = _i8(5000, 8192, 9)
    save_fni8(path, ts, shards={"pp_stages": [["big", "lm_head.weight"]]})
    got = load_fni8_checkpoint(path, device="cuda")
    for name, obj in ts.items():
        ref = obj if isinstance(obj, QTensor) else QTensor(obj, None, scheme="raw")
        assert got[name].data.is_cuda
        _same(got[name].to("cpu"), ref)
    part = load_fni8_checkpoint(path, device="cuda", shard="pp:0")
    assert set(part) == {"big", "lm_head.weight"}
    _same(part["big"].to("cpu"), ts["big"])


@pytest.mark.gpu
def test_loaded_weights_give_bitwise_linear(tmp_path):
    """save -> load is byte-exact, so the W8A8 linear on loaded weights equals the
    one on the weights it was built from, bit for bit (the reference's
    tests/test_convert.py:120-136 check at the linear)."""
    from fni8serve_amd import linear
    path = str(tmp_path / "m.fni8")
    ts = {"qkv": _i8(6144, 4096, 1), "down": _i8(4096, 12288, 2)}
    bias = torch.randn(6144).half()
    save_fni8(path, dict(ts, **{"qkv.bias": bias}))
    sd = load_fni8_state_dict(path, device="cuda")
    g = torch.Generator().manual_seed(5)
    for M in (1, 4, 64, 512):
        for name, K in (("qkv", 4096), ("down", 12288)):
            x = torch.randn(M, K, generator=g).half().cuda()
            b = sd["qkv.bias"] if name == "qkv" else None
            y_loaded = linear(x, sd[name], b)
            y_direct = linear(x, ts[name].to("cuda"), None if b is None else bias.cuda())
            assert torch.equal(y_loaded, y_direct), (name, M)
