"""Checkpoint loading for the MoE path: safetensors shards -> HbmExpertStore
(routed FP4 experts, the MTP block's experts, the FP8 shared experts) and
the per-layer weights the FFN reads.

CheckpointIndex follows WeightLoader (weight_loader.py:48-134): the key ->
shard map comes from model.safetensors.index.json when present, else from
scanning the directory's *.safetensors files; tensors are read through
safetensors' memory-mapped safe_open.  Keys are the reference's:
  layers.{L}.ffn.experts.{E}.w{1,3,2}.{weight,scale}      engine.py:1090-1093
  mtp.0.ffn.experts.{E}.w{1,3,2}.{weight,scale}           engine.py:1900-1915
  layers.{L}.ffn.shared_experts.w{1,3,2}.{weight,scale}   engine.py:1747-1750
  layers.{L}.ffn.gate.{weight,scale,bias,tid2eid}, layers.{L}.ffn_norm.weight
                                                          engine.py:470-510
  mtp.0.ffn.gate.{weight,bias}, mtp.0.{enorm,hnorm,norm,ffn_norm}.weight
                                                          engine.py:1864-1872
  embed.weight, head.weight, norm.weight                  engine.py:426-443
Routed experts keep their bytes: int8 packed e2m1 and E8M0 scales (one byte
each; fp32 scales must be exact powers of two).  Shared-expert scales of one
byte are UE8M0 and become fp32 as _ue8m0_to_f32 does (weight_loader.py:14-19:
the byte shifted into an fp32 exponent).  An expert the checkpoint lacks is
marked absent in the store (its table row is zero: skipped, as the
reference skips a loader returning None).
"""
from __future__ import annotations

import json
import os
from collections import defaultdict

import torch

from .expert_store import HbmExpertStore

_PARTS = ("w1.weight", "w1.scale", "w3.weight", "w3.scale", "w2.weight", "w2.scale")


class CheckpointIndex:
    """Key -> shard map of a safetensors checkpoint directory; memory-mapped reads."""

    def __init__(self, weight_dir: str):
        from safetensors import safe_open
        self._safe_open = safe_open
        self.weight_dir = weight_dir
        self.weight_map: dict[str, str] = {}
        self._open: dict[str, object] = {}
        idx_path = os.path.join(weight_dir, "model.safetensors.index.json")
        if os.path.exists(idx_path):
            with open(idx_path) as f:
                self.weight_map = dict(json.load(f)["weight_map"])
        else:
            for fname in sorted(os.listdir(weight_dir)):
                if fname.endswith(".safetensors"):
                    with safe_open(os.path.join(weight_dir, fname), framework="pt", device="cpu") as f:
                        for key in f.keys():
                            self.weight_map[key] = fname

    def _shard(self, fname: str):
        if fname not in self._open:
            self._open[fname] = self._safe_open(os.path.join(self.weight_dir, fname), framework="pt", device="cpu")
        return self._open[fname]

    def __contains__(self, key: str) -> bool:
        return key in self.weight_map

    def keys(self):
        return self.weight_map.keys()

    def get_weight(self, key: str):
        fname = self.weight_map.get(key)
        return None if fname is None else self._shard(fname).get_tensor(key)

    def get_weights(self, *keys) -> dict:
        by_file = defaultdict(list)
        for k in keys:
            if k in self.weight_map:
                by_file[self.weight_map[k]].append(k)
        out = {}
        for fname, ks in by_file.items():
            f = self._shard(fname)
            for k in ks:
                out[k] = f.get_tensor(k)
        return out

    def close(self) -> None:
        self._open.clear()


def expert_keys(prefix: str) -> list[str]:
    return [f"{prefix}.{p}" for p in _PARTS]


def checkpoint_shape(index: CheckpointIndex) -> dict:
    """n_layers, n_experts, d, i (from the routed experts' keys and w1's shape) and whether an MTP block exists."""
    layers, experts = set(), set()
    first = None
    for k in index.keys():
        parts = k.split(".")
        if len(parts) >= 6 and parts[0] == "layers" and parts[2] == "ffn" and parts[3] == "experts":
            layers.add(int(parts[1]))
            experts.add(int(parts[4]))
            if first is None and k.endswith(".w1.weight"):
                first = k
    if first is None:
        raise ValueError(f"no routed experts (layers.L.ffn.experts.E.*) in {index.weight_dir}")
    w1 = index.get_weight(first)
    i, d_half = w1.shape
    return {"n_layers": max(layers) + 1, "n_experts": max(experts) + 1, "d": 2 * d_half, "i": i,
            "mtp": any(k.startswith("mtp.0.ffn.experts.") for k in index.keys())}


def _e8m0_bytes(scale: torch.Tensor) -> torch.Tensor:
    """E8M0 scale bytes of an FP4 weight's scales.  float8_e8m0fnu scales are
    their bytes.  Every other dtype is taken by value, as the reference's
    loaders do (scale.to(torch.float32), engine.py:1066-1080,
    weight_loader.py:40-44), so a uint8 or int8 scale of 127 means 127.0, not
    2^0; those values are stored as their exponent byte when they are exact
    positive powers of two (2^(e-127), e in 1..254), and refused otherwise:
    the store holds E8M0 exponents only."""
    if scale.dtype == torch.float8_e8m0fnu:
        return scale.view(torch.uint8)
    f = scale.to(torch.float32)
    bits = f.view(torch.int32)
    exp = (bits >> 23) & 0xFF
    if bool(((bits & 0x807FFFFF) != 0).any()) or bool(((exp == 0) | (exp == 255)).any()):
        raise ValueError(f"FP4 scales of dtype {scale.dtype} are taken by value and must then be positive powers "
                         "of two to be stored as E8M0 exponents (other scales: pass the weights as fp32-scale "
                         "tuples to FusedMoEFFN.forward instead)")
    return exp.to(torch.uint8)


def _ue8m0_to_f32(scale: torch.Tensor) -> torch.Tensor:
    """weight_loader.py:14-19: one-byte scales shifted into an fp32 exponent; wider scales by value."""
    if scale.element_size() != 1:
        return scale.to(torch.float32)
    return (scale.view(torch.uint8).to(torch.int32) << 23).view(torch.float32)


def _copy_expert(store: HbmExpertStore, layer: int, eid: int, t: dict, prefix: str) -> bool:
    keys = expert_keys(prefix)
    if keys[0] not in t:
        store.mark_absent(layer, eid)
        return False
    views = store.expert_views(layer, eid)
    for j, (view, key) in enumerate(zip(views, keys)):
        src = t.get(key)
        if src is None:
            raise ValueError(f"{key} missing while {keys[0]} is present")
        if tuple(src.shape) != tuple(view.shape):
            raise ValueError(f"{key}: shape {tuple(src.shape)}, the store holds {tuple(view.shape)}")
        if j % 2 == 0 and src.element_size() != 1:
            raise ValueError(f"{key}: packed FP4 data must be int8/uint8, got {src.dtype}")
        view.view(torch.uint8).copy_(src.view(torch.uint8) if j % 2 == 0 else _e8m0_bytes(src))
    return True


def _copy_shared(store: HbmExpertStore, layer: int, t: dict, prefix: str) -> bool:
    keys = expert_keys(prefix)
    if keys[0] not in t:
        store.mark_no_shared(layer)
        return False
    views = store.shared_views(layer)
    for j, (view, key) in enumerate(zip(views, keys)):
        src = t.get(key)
        if src is None:
            raise ValueError(f"{key} missing while {keys[0]} is present")
        if tuple(src.shape) != tuple(view.shape):
            raise ValueError(f"{key}: shape {tuple(src.shape)}, the store holds {tuple(view.shape)}")
        if j % 2 == 0:
            if src.dtype not in (torch.float8_e4m3fn, torch.uint8):
                raise ValueError(f"{key}: the shared expert must be FP8 e4m3, got {src.dtype}")
            view.view(torch.uint8).copy_(src.view(torch.uint8))
        else:
            view.copy_(_ue8m0_to_f32(src))
    return True


def load_expert_store(index: CheckpointIndex, device="cuda", shape: dict | None = None, with_mtp: bool = True,
                      log=None) -> HbmExpertStore:
    """Every routed expert (store layer L), the MTP block's experts (store layer
    n_layers, when present and with_mtp) and the shared experts, copied into
    one HbmExpertStore."""
    shape = checkpoint_shape(index) if shape is None else shape
    n_layers, n_exp, d, i = shape["n_layers"], shape["n_experts"], shape["d"], shape["i"]
    mtp = with_mtp and shape.get("mtp", False)
    store = HbmExpertStore(n_layers + (1 if mtp else 0), n_exp, d, i, device, with_shared=True)
    for layer in range(n_layers + (1 if mtp else 0)):
        base = f"layers.{layer}.ffn" if layer < n_layers else "mtp.0.ffn"
        for eid in range(n_exp):
            prefix = f"{base}.experts.{eid}"
            _copy_expert(store, layer, eid, index.get_weights(*expert_keys(prefix)), prefix)
        prefix = f"{base}.shared_experts"
        _copy_shared(store, layer, index.get_weights(*expert_keys(prefix)), prefix)
        if log is not None:
            log(f"layer {layer} loaded")
    return store


def _bf16_weight(index: CheckpointIndex, key: str, device, scale_key: str | None = None) -> torch.Tensor | None:
    """_deq (engine.py:625-646) for the dense weights the FFN path reads: bf16 as
    is; e4m3 with 128x128 block scales as load_fp8_weight (weight_loader.py:22-32);
    anything else cast to bf16."""
    w = index.get_weight(key)
    if w is None:
        return None
    if w.dtype == torch.float8_e4m3fn:
        scale = index.get_weight(scale_key) if scale_key else None
        x = w.to(torch.float32)
        if scale is not None:
            sf = _ue8m0_to_f32(scale).repeat_interleave(128, 0).repeat_interleave(128, 1)
            x = x * sf[: x.shape[0], : x.shape[1]]
        w = x
    return w.to(torch.bfloat16).to(device)


def load_layer_weights(index: CheckpointIndex, layer: int, device, prefix: str | None = None) -> dict:
    """The FFN-side layer weights under the reference's short keys: ffn.gate.weight
    (bf16), ffn.gate.bias (fp32), ffn.gate.tid2eid (int64), ffn_norm.weight (bf16)."""
    prefix = f"layers.{layer}" if prefix is None else prefix
    lw = {}
    gate = _bf16_weight(index, f"{prefix}.ffn.gate.weight", device, f"{prefix}.ffn.gate.scale")
    if gate is not None:
        lw["ffn.gate.weight"] = gate
    bias = index.get_weight(f"{prefix}.ffn.gate.bias")
    if bias is not None:
        lw["ffn.gate.bias"] = bias.to(torch.float32).to(device)
    tid = index.get_weight(f"{prefix}.ffn.gate.tid2eid")
    if tid is not None:
        lw["ffn.gate.tid2eid"] = tid.to(torch.int64).contiguous().to(device)
    norm = index.get_weight(f"{prefix}.ffn_norm.weight")
    if norm is not None:
        lw["ffn_norm.weight"] = norm.to(torch.bfloat16).to(device)
    return lw


def select_lm_head(index: CheckpointIndex, config, embed, device):
    """The lm_head as the reference picks it (engine.py:431-443): the embedding
    when tie_word_embeddings is set and an embedding exists; else head.weight,
    else output.weight, else the embedding (None when there is none)."""
    if getattr(config, "tie_word_embeddings", False) and embed is not None:
        return embed
    for key in ("head", "output"):
        w = _bf16_weight(index, f"{key}.weight", device, f"{key}.scale")
        if w is not None:
            return w
    return embed


def load_engine(weight_dir: str, config=None, device="cuda", with_mtp: bool = True, log=None):
    """A HomeSeekMoEEngine over a checkpoint: the expert store, the FFN layer
    weights, embed / lm_head (select_lm_head) / final
    norm, and the MTP block's FFN weights and norms when present."""
    from .engine import HomeSeekMoEEngine
    from .model_config import MoEConfig
    index = CheckpointIndex(weight_dir)
    shape = checkpoint_shape(index)
    if config is None:
        config = MoEConfig(num_hidden_layers=shape["n_layers"], hidden_size=shape["d"],
                           moe_intermediate_size=shape["i"], n_routed_experts=shape["n_experts"])
    store = load_expert_store(index, device, shape, with_mtp, log)
    lws = {l: load_layer_weights(index, l, device) for l in range(shape["n_layers"])}
    embed = _bf16_weight(index, "embed.weight", device)
    head = select_lm_head(index, config, embed, device)
    norm = _bf16_weight(index, "norm.weight", device)
    mtp = None
    if with_mtp and shape["mtp"]:
        mtp = {"layer": load_layer_weights(index, shape["n_layers"], device, prefix="mtp.0"),
               "layer_idx": shape["n_layers"]}
        for n in ("enorm", "hnorm", "norm"):
            w = _bf16_weight(index, f"mtp.0.{n}.weight", device)
            if w is not None:
                mtp[f"{n}.weight"] = w
    index.close()
    return HomeSeekMoEEngine(config, store, lws, lm_head=head, norm_weight=norm,
                             embed=embed, mtp_weights=mtp)
