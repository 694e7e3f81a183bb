"""The safetensors checkpoint loader (CPU): a small checkpoint written here in
the reference's key layout, split over two shards with an index file, loads
into the expert store byte for byte; absent experts and a layer without a
shared expert are marked; UE8M0 shared scales become 2^(e-127) fp32 values
(the reference's shift into the exponent); fp32 power-of-two FP4 scales become
E8M0 bytes and other fp32 scales are refused; the layer weights, MTP block and
head/embed fallback come through under the reference's short keys."""
import json

import pytest
import torch
from safetensors.torch import save_file

from home_seek_amd import checkpoint

NL, E, D, I, K, V = 2, 4, 256, 128, 2, 64


def fp4_expert(g, scale_fp32=False):
    t = {}
    for w, (r, c) in (("w1", (I, D)), ("w3", (I, D)), ("w2", (D, I))):
        t[f"{w}.weight"] = torch.randint(-128, 128, (r, c // 2), generator=g, dtype=torch.int8)
        e = torch.randint(119, 125, (r, c // 32), generator=g, dtype=torch.uint8)
        t[f"{w}.scale"] = torch.ldexp(torch.ones(r, c // 32), e.to(torch.int32) - 127) if scale_fp32 else \
            e.view(torch.float8_e8m0fnu)
    return t


def fp8_shared(g):
    t = {}
    for w, (r, c) in (("w1", (I, D)), ("w3", (I, D)), ("w2", (D, I))):
        t[f"{w}.weight"] = torch.randint(0, 126, (r, c), generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn)
        t[f"{w}.scale"] = torch.randint(110, 130, (r // 128, c // 128), generator=g, dtype=torch.uint8).view(
            torch.float8_e8m0fnu)
    return t


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    g = torch.Generator().manual_seed(1)
    d = tmp_path_factory.mktemp("ckpt")
    tensors = {}
    for l in range(NL):
        for e in range(E):
            if (l, e) == (1, 2):
                continue  # absent expert
            for k, v in fp4_expert(g, scale_fp32=(l, e) == (0, 3)).items():
                tensors[f"layers.{l}.ffn.experts.{e}.{k}"] = v
        if l == 0:
            for k, v in fp8_shared(g).items():
                tensors[f"layers.{l}.ffn.shared_experts.{k}"] = v
        tensors[f"layers.{l}.ffn.gate.weight"] = torch.randn(E, D, generator=g).to(torch.bfloat16)
        tensors[f"layers.{l}.ffn.gate.bias"] = torch.randn(E, generator=g)
        tensors[f"layers.{l}.ffn_norm.weight"] = torch.randn(D, generator=g)  # fp32: loaded as bf16
    tensors["layers.0.ffn.gate.tid2eid"] = torch.randint(0, E, (V, K), generator=g, dtype=torch.int32)
    for e in range(E):
        for k, v in fp4_expert(g).items():
            tensors[f"mtp.0.ffn.experts.{e}.{k}"] = v
    for k, v in fp8_shared(g).items():
        tensors[f"mtp.0.ffn.shared_experts.{k}"] = v
    q = torch.randint(0, 126, (E, D), generator=g, dtype=torch.uint8).view(torch.float8_e4m3fn)
    tensors["mtp.0.ffn.gate.weight"] = q
    tensors["mtp.0.ffn.gate.scale"] = torch.tensor([[127, 126]], dtype=torch.uint8).view(torch.float8_e8m0fnu)
    for n in ("enorm", "hnorm", "norm"):
        tensors[f"mtp.0.{n}.weight"] = torch.randn(D, generator=g).to(torch.bfloat16)
    tensors["embed.weight"] = torch.randn(V, D, generator=g).to(torch.bfloat16)
    tensors["norm.weight"] = torch.randn(D, generator=g).to(torch.bfloat16)
    keys = sorted(tensors)
    shards = {"model-00001-of-00002.safetensors": keys[: len(keys) // 2],
              "model-00002-of-00002.safetensors": keys[len(keys) // 2:]}
    wmap = {}
    for fname, ks in shards.items():
        save_file({k: tensors[k].contiguous() for k in ks}, str(d / fname))
        wmap.update({k: fname for k in ks})
    (d / "model.safetensors.index.json").write_text(json.dumps({"metadata": {"total_size": 0}, "weight_map": wmap}))
    return str(d), tensors


def test_store_holds_the_checkpoint_bytes(ckpt):
    path, t = ckpt
    index = checkpoint.CheckpointIndex(path)
    shape = checkpoint.checkpoint_shape(index)
    assert shape == {"n_layers": NL, "n_experts": E, "d": D, "i": I, "mtp": True}
    store = checkpoint.load_expert_store(index, "cpu", shape)
    assert store.n_layers == NL + 1
    for l in range(NL + 1):
        base = f"layers.{l}.ffn" if l < NL else "mtp.0.ffn"
        for e in range(E):
            if (l, e) == (1, 2):
                assert not store.has_expert(l, e)
                assert int(store.table(l)[e].abs().sum()) == 0
                continue
            assert store.has_expert(l, e)
            for view, key in zip(store.expert_views(l, e), checkpoint.expert_keys(f"{base}.experts.{e}")):
                src = t[key]
                if src.dtype == torch.float32:  # power-of-two fp32 scales -> E8M0 exponent bytes
                    want = ((src.view(torch.int32) >> 23) & 0xFF).to(torch.uint8)
                else:
                    want = src.view(torch.uint8)
                assert torch.equal(view.view(torch.uint8), want), key
        if l == 1:
            assert not store.has_shared(l) and store.shared_entry(l) is None
            continue
        for view, key in zip(store.shared_views(l), checkpoint.expert_keys(f"{base}.shared_experts")):
            src = t[key]
            if key.endswith(".scale"):
                e = src.view(torch.uint8).to(torch.float64)
                assert torch.equal(view.to(torch.float64), torch.pow(2.0, e - 127)), key
            else:
                assert torch.equal(view.view(torch.uint8), src.view(torch.uint8)), key


def test_layer_weights_mtp_and_head(ckpt):
    path, t = ckpt
    eng = checkpoint.load_engine(path, device="cpu")
    lw0 = eng._get_layer_weights(0)
    assert torch.equal(lw0["ffn.gate.weight"], t["layers.0.ffn.gate.weight"])
    assert lw0["ffn.gate.bias"].dtype == torch.float32
    assert lw0["ffn.gate.tid2eid"].dtype == torch.int64
    assert torch.equal(lw0["ffn.gate.tid2eid"], t["layers.0.ffn.gate.tid2eid"].long())
    assert torch.equal(lw0["ffn_norm.weight"], t["layers.0.ffn_norm.weight"].to(torch.bfloat16))
    assert "ffn.gate.tid2eid" not in eng._get_layer_weights(1)
    assert eng.lm_head is eng.embed  # no head.weight: the tied embedding (engine.py:426-443)
    mw = eng._mtp_weights
    assert mw["layer_idx"] == NL and set(mw) >= {"enorm.weight", "hnorm.weight", "norm.weight", "layer"}
    # an e4m3 gate with UE8M0 128x128 block scales (load_fp8_weight): scale 2^0 then 2^-1 by column block
    gq = t["mtp.0.ffn.gate.weight"].to(torch.float32)
    want = torch.cat([gq[:, :128], gq[:, 128:] * 0.5], dim=1).to(torch.bfloat16)
    assert torch.equal(mw["layer"]["ffn.gate.weight"], want)
    assert eng._load_expert_fp4_raw(1, 2) is None and eng._load_expert_weights(1, 2) is None
    assert eng._get_shared_expert(1) is None


def test_loader_refuses_what_the_store_cannot_hold(tmp_path):
    g = torch.Generator().manual_seed(2)
    t = {f"layers.0.ffn.experts.0.{k}": v for k, v in fp4_expert(g).items()}
    t["layers.0.ffn.experts.0.w1.scale"] = torch.full((I, D // 32), 0.3)
    save_file(t, str(tmp_path / "a.safetensors"))
    index = checkpoint.CheckpointIndex(str(tmp_path))
    with pytest.raises(ValueError, match="powers of two"):
        checkpoint.load_expert_store(index, "cpu")
