"""`mtp.load(ck, full_cfg, tp, dev, dtype, max_batch, kv_rows)` on a checkpoint written in the
real model's tensor names: every tensor lands where `attach` puts its random twin, the loaded
head drafts the same tokens, and the flag / missing-head / shape cases behave like
`mtp.py:131-190` (None, None, error)."""

from __future__ import annotations

import pytest
import torch
from safetensors.torch import save_file

import mtp
import verify_model as vm
from tests import model_helpers as mh
from weights import Checkpoint


def hf_tensors(m: mtp.MTP, cfg: vm.Cfg) -> dict[str, torch.Tensor]:
    """The MTP head under the checkpoint's names: fused tensors split back into the parts the
    checkpoint stores (router rows / shared gate row, shared gate / up), experts one by one."""
    w, i, si = m.weights, cfg.inter, cfg.shared_inter
    out = {"mtp.fc.weight": m.fc, "mtp.pre_fc_norm_embedding.weight": m.pre_fc_norm_embedding,
           "mtp.pre_fc_norm_hidden.weight": m.pre_fc_norm_hidden, "mtp.norm.weight": m.norm}
    p = "mtp.layers.0"
    out[f"{p}.input_layernorm.weight"] = w["in_norm"]
    out[f"{p}.post_attention_layernorm.weight"] = w["post_norm"]
    for name in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm"):
        out[f"{p}.self_attn.{name}.weight"] = w[name]
    out[f"{p}.mlp.gate.weight"] = w["router_gate"][: cfg.experts]
    out[f"{p}.mlp.shared_expert_gate.weight"] = w["router_gate"][cfg.experts :]
    out[f"{p}.mlp.shared_expert.gate_proj.weight"] = w["shared_gate_up"][:si]
    out[f"{p}.mlp.shared_expert.up_proj.weight"] = w["shared_gate_up"][si:]
    out[f"{p}.mlp.shared_expert.down_proj.weight"] = w["shared_down"]
    ex = w["experts"]
    for e in range(cfg.experts):
        q = f"{p}.mlp.experts.{e}"
        for suffix, key in (("weight", ""), ("weight_scale", "_scale")):
            if f"gate_up{key}" not in ex:
                continue
            out[f"{q}.gate_proj.{suffix}"] = ex[f"gate_up{key}"][e, :i]
            out[f"{q}.up_proj.{suffix}"] = ex[f"gate_up{key}"][e, i:]
            out[f"{q}.down_proj.{suffix}"] = ex[f"down{key}"][e]
    return {k: v.contiguous().clone() for k, v in out.items()}


@pytest.fixture()
def served(monkeypatch):
    monkeypatch.setenv("SEED_MTP_SERVE", "1")
    monkeypatch.delenv("SEED_MTP", raising=False)


def write(tmp_path, tensors, shards=2):
    names = sorted(tensors)
    for s in range(shards):
        save_file({n: tensors[n] for n in names[s::shards]}, str(tmp_path / f"model-{s}.safetensors"))
    return Checkpoint(tmp_path)


@pytest.mark.parametrize("experts", ["quantized", "dense"])
def test_round_trip_matches_attach(tmp_path, served, experts):
    model = mh.build("cpu", k=mtp.MTP_K, mtp_experts=experts)
    ref = model.mtp
    ck = write(tmp_path, hf_tensors(ref, model.cfg))
    got = mtp.load(ck, model.cfg, None, "cpu", torch.float32, 2, model.blocks.rows)
    assert got is not None and got.k == mtp.MTP_K
    for name in ("fc", "pre_fc_norm_embedding", "pre_fc_norm_hidden", "norm"):
        assert torch.equal(getattr(got, name), getattr(ref, name)), name
    assert sorted(got.weights) == sorted(ref.weights)
    for name, ten in ref.weights.items():
        if name == "experts":
            assert sorted(got.weights[name]) == sorted(ten)
            for key, part in ten.items():
                # MXFP4 payloads stay uint8; dense experts take the load dtype
                want_dt = torch.uint8 if part.dtype == torch.uint8 else torch.float32
                assert got.weights[name][key].dtype == want_dt
                assert torch.equal(got.weights[name][key], part.to(want_dt)), key
        else:
            assert torch.equal(got.weights[name], ten), name
    for key in ("k", "v"):
        assert got.pool[key].shape == ref.pool[key].shape and not got.pool[key].any()

    if experts == "dense":
        return
    # the loaded head drafts what the attached one drafts
    prompt = mh.prompts(1)[0]
    logits = model.prefill(0, prompt)
    base = int(logits.argmax())
    hidden = model.hidden_cache[:1].clone()
    got.pool["k"].copy_(ref.pool["k"])  # the prompt's MTP cache rows
    got.pool["v"].copy_(ref.pool["v"])
    want = mtp.draft(model, ref, hidden, [base], [0], [len(prompt)])
    assert mtp.draft(model, got, hidden, [base], [0], [len(prompt)]) == want


def test_flag_off_or_no_head_gives_none(tmp_path, monkeypatch):
    model = mh.build("cpu")
    tensors = hf_tensors(model.mtp, model.cfg)
    ck = write(tmp_path, tensors, shards=1)
    monkeypatch.delenv("SEED_MTP_SERVE", raising=False)
    monkeypatch.delenv("SEED_MTP", raising=False)
    assert mtp.load(ck, model.cfg, None, "cpu", torch.float32, 2, model.blocks.rows) is None
    monkeypatch.setenv("SEED_MTP", "1")  # the older alias turns it on too
    assert mtp.load(ck, model.cfg, None, "cpu", torch.float32, 2, model.blocks.rows) is not None
    other = tmp_path / "nohead"
    other.mkdir()
    del tensors["mtp.fc.weight"]
    assert mtp.load(write(other, tensors, 1), model.cfg, None, "cpu", torch.float32, 2,
                    model.blocks.rows) is None


def test_shape_and_argument_errors(tmp_path, served):
    model = mh.build("cpu")
    tensors = hf_tensors(model.mtp, model.cfg)
    tensors["mtp.layers.0.self_attn.k_proj.weight"] = tensors["mtp.layers.0.self_attn.k_proj.weight"][:-1]
    ck = write(tmp_path, tensors, 1)
    with pytest.raises(ValueError, match="k_proj"):
        mtp.load(ck, model.cfg, None, "cpu", torch.float32, 2, model.blocks.rows)
    with pytest.raises(ValueError, match="kv_rows"):
        mtp.load(ck, model.cfg, None, "cpu", torch.float32, 2, model.cfg.block_size + 1)
    with pytest.raises(ValueError, match="max_batch"):
        mtp.load(ck, model.cfg, None, "cpu", torch.float32, 0, model.blocks.rows)

    class TwoRanks:
        world = 2

    with pytest.raises(ValueError, match="one GPU"):
        mtp.load(ck, model.cfg, TwoRanks(), "cpu", torch.float32, 2, model.blocks.rows)
