"""The checkpoint reader (`weights.py`) on synthetic safetensors shards, on the CPU.

The shards are written with the `safetensors` library under the real checkpoint's per-expert
names, split over two files the way the reference tests split theirs
(`test_seed_parity.py:72-93`): `{prefix}.experts.{e}.{gate_proj|up_proj|down_proj}.weight`,
plus `.weight_scale` for MXFP4. The header parser is checked against the library's own reader,
and `load_experts` against the stacking rule `gate_up = cat(gate, up)` (`model.py:758-804`).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

import weights
from tests.moe_inputs import random_experts

E, H, I = 6, 64, 32
PREFIX = "model.language_model.layers.0.mlp"


def _write_shards(path, tensors: dict[str, torch.Tensor]) -> None:
    keys = sorted(tensors)
    for i, part in enumerate((keys[::2], keys[1::2])):
        save_file({k: tensors[k].contiguous() for k in part}, str(path / f"model-{i}.safetensors"))


def _mxfp4_tensors(seed: int = 0) -> tuple[dict[str, torch.Tensor], dict[str, np.ndarray]]:
    ex = random_experts(E, H, I, seed=seed)
    t: dict[str, torch.Tensor] = {}
    for e in range(E):
        for proj, rows in (("gate_proj", slice(0, I)), ("up_proj", slice(I, 2 * I))):
            t[f"{PREFIX}.experts.{e}.{proj}.weight"] = torch.from_numpy(ex["gate_up"][e, rows].copy())
            t[f"{PREFIX}.experts.{e}.{proj}.weight_scale"] = torch.from_numpy(ex["gate_up_scale"][e, rows].copy())
        t[f"{PREFIX}.experts.{e}.down_proj.weight"] = torch.from_numpy(ex["down"][e].copy())
        t[f"{PREFIX}.experts.{e}.down_proj.weight_scale"] = torch.from_numpy(ex["down_scale"][e].copy())
    t["model.language_model.embed_tokens.weight"] = torch.randn(50, H).to(torch.bfloat16)
    t["model.language_model.norm.weight"] = torch.randn(H)
    t["lm_head.bias_count"] = torch.arange(7, dtype=torch.int64)
    t["flags"] = torch.tensor([True, False, True])
    return t, ex


def test_headers_match_the_library_reader(tmp_path) -> None:
    tensors, _ = _mxfp4_tensors()
    _write_shards(tmp_path, tensors)
    ck = weights.Checkpoint(tmp_path)
    assert ck.names() == sorted(tensors)
    for f in ck.files:
        with safe_open(str(f), framework="pt") as lib:
            for name in lib.keys():
                want = lib.get_tensor(name)
                got = ck.load(name, "cpu")
                assert got.dtype == want.dtype and got.shape == want.shape, name
                assert torch.equal(got, want), name
    assert ck.has("flags") and not ck.has("missing")
    with pytest.raises(KeyError):
        ck.load("missing", "cpu")


def test_load_casts_on_request(tmp_path) -> None:
    tensors, _ = _mxfp4_tensors()
    _write_shards(tmp_path, tensors)
    ck = weights.Checkpoint(tmp_path)
    got = ck.load("model.language_model.norm.weight", "cpu", torch.bfloat16)
    assert got.dtype == torch.bfloat16
    assert torch.equal(got, tensors["model.language_model.norm.weight"].to(torch.bfloat16))


@pytest.mark.parametrize("start,count", [(0, E), (2, 3), (5, 1)])
def test_load_experts_stacks_the_mxfp4_layout(tmp_path, start, count) -> None:
    tensors, ex = _mxfp4_tensors(seed=3)
    _write_shards(tmp_path, tensors)
    ck = weights.Checkpoint(tmp_path)
    got = weights.load_experts(ck, PREFIX, weights.Shard(start, count), "cpu", torch.bfloat16)
    assert set(got) == {"gate_up", "gate_up_scale", "down", "down_scale"}
    sl = slice(start, start + count)
    for key in got:
        assert got[key].dtype == torch.uint8, key  # payloads and scales stay uint8
        np.testing.assert_array_equal(got[key].numpy(), ex[key][sl], err_msg=key)
    # gate rows first, then up rows, per expert
    e = start
    np.testing.assert_array_equal(got["gate_up"][0, :I].numpy(),
                                  tensors[f"{PREFIX}.experts.{e}.gate_proj.weight"].numpy())
    np.testing.assert_array_equal(got["gate_up"][0, I:].numpy(),
                                  tensors[f"{PREFIX}.experts.{e}.up_proj.weight"].numpy())


def test_load_experts_casts_a_dense_checkpoint(tmp_path) -> None:
    g = torch.Generator().manual_seed(0)
    t = {}
    for e in range(E):
        for proj, shape in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I))):
            t[f"mtp.layers.0.mlp.experts.{e}.{proj}.weight"] = torch.randn(*shape, generator=g)
    _write_shards(tmp_path, t)
    ck = weights.Checkpoint(tmp_path)
    got = weights.load_experts(ck, "mtp.layers.0.mlp", weights.Shard(0, E), "cpu", torch.bfloat16)
    assert set(got) == {"gate_up", "down"}
    for e in range(E):
        want = torch.cat([t[f"mtp.layers.0.mlp.experts.{e}.gate_proj.weight"],
                          t[f"mtp.layers.0.mlp.experts.{e}.up_proj.weight"]]).to(torch.bfloat16)
        assert got["gate_up"].dtype == torch.bfloat16
        assert torch.equal(got["gate_up"][e], want)
        assert torch.equal(got["down"][e], t[f"mtp.layers.0.mlp.experts.{e}.down_proj.weight"].to(torch.bfloat16))


def test_shard_rows() -> None:
    sh = weights.Shard(3, 2)
    assert sh.stop == 5 and sh.rows(4) == slice(12, 20)


def test_errors(tmp_path) -> None:
    with pytest.raises(FileNotFoundError):
        weights.Checkpoint(tmp_path)
    tensors, _ = _mxfp4_tensors()
    # expert 4's down_proj has another shape: it cannot stack
    tensors[f"{PREFIX}.experts.4.down_proj.weight"] = torch.zeros(H, I // 2 + 1, dtype=torch.uint8)
    _write_shards(tmp_path, tensors)
    ck = weights.Checkpoint(tmp_path)
    with pytest.raises(ValueError, match="experts.4.down_proj"):
        weights.load_experts(ck, PREFIX, weights.Shard(0, E), "cpu", torch.bfloat16)
    with pytest.raises(KeyError):
        weights.load_experts(ck, PREFIX, weights.Shard(0, E + 1), "cpu", torch.bfloat16)


def test_truncated_shard(tmp_path) -> None:
    """A data section shorter than the header's byte ranges is refused when the shard is
    indexed; a shard cut after indexing gives a short read, not a partial tensor."""
    f = tmp_path / "model-0.safetensors"
    save_file({"a": torch.arange(1000, dtype=torch.int64)}, str(f))
    whole = f.read_bytes()
    f.write_bytes(whole[:-100])
    with pytest.raises(ValueError, match="byte range"):
        weights.Checkpoint(tmp_path)
    f.write_bytes(whole)
    ck = weights.Checkpoint(tmp_path)
    f.write_bytes(whole[:-100])
    with pytest.raises(OSError, match="short read"):
        ck.load("a", "cpu")


def test_header_checks(tmp_path) -> None:
    """Sizes that disagree with shape x dtype, unknown dtypes and names present in two shards are
    format errors."""
    import json as _json

    def shard(name, table, data):
        head = _json.dumps(table).encode()
        (tmp_path / name).write_bytes(len(head).to_bytes(8, "little") + head + data)

    shard("a.safetensors", {"x": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, bytes(12))
    with pytest.raises(ValueError, match="byte range"):
        weights.Checkpoint(tmp_path)
    shard("a.safetensors", {"x": {"dtype": "Q9", "shape": [3], "data_offsets": [0, 12]}}, bytes(12))
    with pytest.raises(ValueError, match="dtype"):
        weights.Checkpoint(tmp_path)
    shard("a.safetensors", {"x": {"dtype": "F32", "shape": [3], "data_offsets": [0, 12]},
                            "__metadata__": {"format": "pt"}}, bytes(12))
    ck = weights.Checkpoint(tmp_path)
    assert ck.names() == ["x"] and ck.info("x").shape == (3,)
    shard("b.safetensors", {"x": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}, bytes(4))
    with pytest.raises(ValueError, match="appears in"):
        weights.Checkpoint(tmp_path)


@pytest.mark.gpu
def test_loaded_experts_run_on_the_device(tmp_path) -> None:
    """The stacked device tensors are the layout the fused MoE reads: the kernel's output on a
    loaded checkpoint equals the fp64 oracle on the source arrays."""
    import mxfp4_gemv
    from oracle import moe_ref
    from tests.moe_inputs import random_routing

    dev = torch.device("cuda:0")
    tensors, ex = _mxfp4_tensors(seed=9)
    _write_shards(tmp_path, tensors)
    got_ex = weights.load_experts(weights.Checkpoint(tmp_path), PREFIX, weights.Shard(0, E), dev,
                                  torch.bfloat16)
    assert all(v.device.type == "cuda" for v in got_ex.values())
    a_e, a_w = random_routing(5, E, 2, seed=10)
    x = np.random.default_rng(11).standard_normal((5, H)).astype(np.float32)
    want = moe_ref.reference_moe(x, ex, a_e, a_w, 2, (0, E))
    got = mxfp4_gemv.fused_moe(torch.from_numpy(x).to(dev), got_ex,
                               (torch.from_numpy(a_e).to(dev), torch.from_numpy(a_w).to(dev)),
                               2, (0, E))
    assert moe_ref.relative_error(got.cpu().numpy(), want) < 1e-5


@pytest.mark.gpu
def test_scale_255_block_fails_at_load(tmp_path, monkeypatch) -> None:
    """A shard holding a 32-element block with e8m0 scale 255 over nonzero codes (which the
    in-register decode gives as NaN, the pinned decode as +-inf) is refused by `load_experts`
    itself, not at its first MoE call. The same block over zero codes loads and runs (its
    pinned decode, 0 * 2^128, is NaN in both decodes), and with `SEED_FUSED_MOE=0` (the torch
    path, which decodes 255 as pinned) the shard loads."""
    import mxfp4_gemv

    dev = torch.device("cuda:0")
    tensors, _ = _mxfp4_tensors(seed=12)
    name = f"{PREFIX}.experts.3.down_proj.weight_scale"
    packed = f"{PREFIX}.experts.3.down_proj.weight"
    tensors[name][7, 0] = 255
    tensors[packed][7, :16] |= 0x11  # nonzero magnitudes in that block
    _write_shards(tmp_path, tensors)
    with pytest.raises(ValueError, match="supports"):
        weights.load_experts(weights.Checkpoint(tmp_path), PREFIX, weights.Shard(0, E), dev,
                             torch.bfloat16)
    monkeypatch.setenv("SEED_FUSED_MOE", "0")
    ex = weights.load_experts(weights.Checkpoint(tmp_path), PREFIX, weights.Shard(0, E), dev,
                              torch.bfloat16)
    assert int(ex["down_scale"][3, 7, 0]) == 255
    monkeypatch.delenv("SEED_FUSED_MOE")

    tensors[packed][7, :16] &= 0x88  # only signed zeros under the 255 scale
    for f in tmp_path.glob("*.safetensors"):
        f.unlink()
    _write_shards(tmp_path, tensors)
    ex = weights.load_experts(weights.Checkpoint(tmp_path), PREFIX, weights.Shard(0, E), dev,
                              torch.bfloat16)
    x = torch.randn(2, H, device=dev).to(torch.bfloat16)
    routing = (torch.tensor([3, 1, 2, 3], dtype=torch.int32, device=dev), torch.full((4,), 0.5, device=dev))
    out = mxfp4_gemv.fused_moe(x, ex, routing, 2, (0, E)).float()
    # the pinned decode of a zero code under scale 255 is 0 * 2^128 = NaN, and both tokens route
    # to expert 3, whose down row 7 holds that block: NaN in hidden column 7 only
    assert torch.isnan(out[:, 7]).all()
    assert torch.isfinite(torch.cat([out[:, :7], out[:, 8:]], dim=1)).all()
