"""The MoE slice of HomeSeekInferenceEngine, on the HBM expert store and HIP kernels.

Method names, arguments and return values follow the reference engine
(src/home_seek/inference_engine/engine.py) so that its _forward_layer, generate
and MTP loop can call them unchanged:
  _load_expert_weights / _load_expert_raw / _load_expert_fp4_raw /
  _load_bf16_deq / _load_expert_deq              engine.py:1084-1335
  _compute_routing_experts / _compute_hash_experts  engine.py:1018-1031
  _get_shared_expert                              engine.py:1779-1849
  _forward_ffn                                    engine.py:1410-1541
  _mtp_verify_batched                             engine.py:2431-2540
  _mtp_generate_draft (stand-in, see below)        engine.py:2251-2339
  decode_step / generate_greedy                    engine.py:2809-2922 (temperature 0)
Attention, mHC, KV caches and sampling stay with the host engine; the hooks
`_snapshot_verify_state` / `_restore_verify_state` are where a full engine
saves and trims its attention state around a verify (no-ops here).
Divergences from the reference, all deliberate:
  * T > 1 uses the same FP4 kernel as T = 1 (the reference switches to a dense
    BF16 union GEMM, fused_moe.py:458-551) and reads each layer's own experts
    (the reference's BF16 cache is keyed by (eid, device) and aliases expert
    e of the first layer that loaded it, engine.py:1319-1323).
  * no host synchronisation inside _forward_ffn (the reference calls .tolist()
    on the routing ids, engine.py:1432-1433); _mtp_verify_batched syncs once,
    decode_step not at all (the acceptance outcome stays on the device).
  * the MTP draft module keeps the reference's data flow (hnorm of the main
    model's last hidden state + enorm of the token embedding, one MoE block
    with the MTP experts, the MTP norm, lm_head, greedy argmax; second draft
    from the first) without its attention and without the e_proj / h_proj
    projections, which are outside the MoE path; its experts are one more
    layer of the HBM store (the checkpoint's mtp.0.ffn.experts.*).
"""
from __future__ import annotations

import warnings

import torch

from . import ops
from ._lib import SCALE_E8M0
from .expert_store import HbmExpertStore
from .fused_moe import FusedMoEFFN, SharedExpertFFN
from .model_config import MoEConfig
from .router import compute_expert_affinity_with_bias


class HomeSeekMoEEngine:
    def __init__(self, config: MoEConfig, store: HbmExpertStore, layer_weights: dict[int, dict],
                 lm_head: torch.Tensor | None = None, norm_weight: torch.Tensor | None = None,
                 embed: torch.Tensor | None = None, mtp_weights: dict | None = None):
        self.config = config
        # mtp_weights: {"hnorm.weight", "enorm.weight", "norm.weight", "layer": layer
        # weights of the MTP block (as for _forward_layer), "layer_idx": its store layer}
        self._mtp_weights = mtp_weights
        self.store = store
        self.device = store.device
        self._layer_weights = layer_weights
        self.lm_head = lm_head
        self.norm_weight = norm_weight
        self.embed = embed
        self._fused_moe = FusedMoEFFN(config.n_routed_experts, config.moe_intermediate_size, config.hidden_size,
                                      config.swiglu_limit)
        self._shared_ffn = SharedExpertFFN(config.hidden_size, config.moe_intermediate_size, config.swiglu_limit)
        self._global_pos = 0
        self._phase = "decode"
        self._last_routed_idx = None

    # ------------------------------------------------------------ weights
    def _get_layer_weights(self, layer_idx: int) -> dict:
        return self._layer_weights[layer_idx]

    @property
    def _last_routed_idx(self):
        """Expert ids [B*T, k] of the last _forward_ffn; a hash layer's are looked
        up (tid2eid[input_ids]) only when read, outside the decode hot path."""
        r = self._last_route
        if isinstance(r, tuple):
            table, ids = r
            return table[ids]
        return r

    @_last_routed_idx.setter
    def _last_routed_idx(self, value):
        self._last_route = value

    def _load_expert_fp4_raw(self, layer_idx: int, eid: int):
        """(w1, w1_scale, w3, w3_scale, w2, w2_scale) device views (E8M0 scales), or None."""
        if not self.store.has_expert(layer_idx, eid):
            return None
        return self.store.expert_views(layer_idx, eid)

    def _load_expert_weights(self, layer_idx: int, eid: int):
        """((w1, s1, fmt), (w3, s3, fmt), (w2, s2, fmt)) with fmt "fp4_gpu" (engine.py:1084-1129).

        As the reference's on-device entries (_make_raw_entry, engine.py:1054-1082),
        the data are the store's int8 views and the scales are fp32 (the E8M0
        values, 2^(e-127), converted by torch's float8_e8m0fnu cast: a new
        tensor of 4 bytes per scale).  The decode kernels read the store's E8M0
        bytes directly through the layer's table, not these entries."""
        raw = self._load_expert_fp4_raw(layer_idx, eid)
        if raw is None:
            return None
        w1, s1, w3, s3, w2, s2 = raw
        return ((w1, s1.to(torch.float32), "fp4_gpu"), (w3, s3.to(torch.float32), "fp4_gpu"),
                (w2, s2.to(torch.float32), "fp4_gpu"))

    _load_expert_raw = _load_expert_weights

    def _load_bf16_deq(self, layer_idx: int, eid: int):
        """BF16 (w1, w3, w2) of this layer's expert, dequantised on demand (no cross-layer alias)."""
        raw = self._load_expert_fp4_raw(layer_idx, eid)
        if raw is None:
            return None
        w1, s1, w3, s3, w2, s2 = raw
        return ops.fp4_dequant_bf16(w1, s1), ops.fp4_dequant_bf16(w3, s3), ops.fp4_dequant_bf16(w2, s2)

    _load_expert_deq = _load_bf16_deq

    def _get_shared_expert(self, layer_idx: int):
        """BF16 (w1, w3, w2) of the FP8 shared expert (load_fp8_weight, weight_loader.py:22-32)."""
        if not self.store.has_shared(layer_idx):
            return None
        views = self.store.shared_views(layer_idx)
        w1, s1, w3, s3, w2, s2 = views
        return ops.fp8_dequant_bf16(w1, s1), ops.fp8_dequant_bf16(w3, s3), ops.fp8_dequant_bf16(w2, s2)

    # ------------------------------------------------------------ routing
    def _compute_hash_experts(self, input_ids: torch.Tensor, layer_idx: int, tid2eid: torch.Tensor):
        """engine.py:1018-1023: ids from the token table, weight 1/k each."""
        B, T = input_ids.shape
        eids = tid2eid[input_ids]
        k = self.config.num_experts_per_tok
        weights = torch.full((B, T, k), 1.0 / k, device=input_ids.device)
        return eids, weights

    def _compute_routing_experts(self, hidden_states, gate_w, gate_bias):
        return compute_expert_affinity_with_bias(hidden_states, gate_w, gate_bias,
                                                 top_k=self.config.num_experts_per_tok,
                                                 routed_scaling_factor=self.config.routed_scaling_factor)

    # ------------------------------------------------------------ FFN
    def _forward_ffn(self, hidden_states: torch.Tensor, lw: dict, layer_idx: int, input_ids=None,
                     out_f32: torch.Tensor | None = None):
        """Router (or hash routing) + routed FP4 experts + FP8 shared expert -> ([B, T, D], set())."""
        gate_w = lw.get("ffn.gate.weight")
        if gate_w is None:
            return torch.zeros_like(hidden_states), set()
        gate_bias = lw.get("ffn.gate.bias")
        tid2eid = lw.get("ffn.gate.tid2eid")
        B, T, D = hidden_states.shape
        flat = hidden_states.reshape(B * T, D)
        hashed = layer_idx < self.config.num_hash_layers and tid2eid is not None and input_ids is not None
        out_bf16 = torch.empty(B * T, D, dtype=torch.bfloat16, device=flat.device)
        if self._one_launch_layer(flat, lw, layer_idx, input_ids, out_f32=out_f32, out_bf16=out_bf16):
            return out_bf16.reshape(B, T, D).to(hidden_states.dtype), set()
        k = self.config.num_experts_per_tok
        table = self.store.table(layer_idx)
        if hashed:
            idx, w = self._compute_hash_experts(input_ids.to(hidden_states.device), layer_idx, tid2eid)
        else:
            idx, w = self._compute_routing_experts(flat, gate_w, gate_bias)
        idx = idx.reshape(B * T, k)
        w = w.reshape(B * T, k)
        self._last_routed_idx = idx
        out = self._fused_moe.forward_table(flat, idx, w, table, SCALE_E8M0,
                                            self.store.shared_entry(layer_idx), out_f32=out_f32)
        return out.reshape(B, T, D).to(hidden_states.dtype), set()

    # the persistent one-launch layer kernel (False: the router and the staged
    # expert kernels, which give the same values and need no co-resident grid)
    use_one_launch_layer = True

    def _one_launch_layer(self, flat: torch.Tensor, lw: dict, layer_idx: int, input_ids=None,
                          out_f32: torch.Tensor | None = None, out_bf16: torch.Tensor | None = None,
                          norm: ops.NormTail | None = None, ids_owned: bool = False) -> bool:
        """The layer's FFN on hidden rows flat [M, D] in one launch when it
        applies (M <= 8, bf16, at most 256 experts): router + routed + shared
        experts (hsmoe_moe_layer_decode), or on hash layers the token table
        looked up in the launch (hsmoe_moe_layer_decode_routed); with `norm`
        the launch also does the next layer's adds + RMSNorm.  ids_owned: the
        caller guarantees input_ids are not rewritten while _last_routed_idx
        may still refer to them (no private copy is made).  -> False (and
        nothing launched) when it does not apply."""
        gate_w = lw.get("ffn.gate.weight")
        if gate_w is None or not self.use_one_launch_layer:
            return False
        tid2eid = lw.get("ffn.gate.tid2eid")
        m = flat.shape[0]
        hashed = layer_idx < self.config.num_hash_layers and tid2eid is not None and input_ids is not None
        k = self.config.num_experts_per_tok
        if (not hashed and m <= ops.MAX_DECODE_TOKENS and gate_w.shape[0] <= ops.MAX_LAYER_EXPERTS
                and flat.dtype == torch.bfloat16 and gate_w.dtype == torch.bfloat16):
            # router + routed + shared experts in one launch (hsmoe_moe_layer_decode)
            _, _, idx, _ = ops.moe_layer_decode(
                flat, gate_w, lw.get("ffn.gate.bias"), self.store.table(layer_idx), SCALE_E8M0,
                self.store.shared_entry(layer_idx), self.config.moe_intermediate_size, k,
                self.config.routed_scaling_factor, self.config.swiglu_limit, out_f32=out_f32, out_bf16=out_bf16,
                norm=norm)
            self._last_routed_idx = idx
            return True
        table = self.store.table(layer_idx)
        if (hashed and m <= ops.MAX_DECODE_TOKENS and table.shape[0] <= ops.MAX_LAYER_EXPERTS
                and flat.dtype == torch.bfloat16 and tid2eid.dtype == torch.int64 and tid2eid.is_contiguous()
                and tid2eid.device == flat.device and input_ids.device == flat.device
                and input_ids.dtype == torch.int64):
            # hash ids (tid2eid[input_ids], weight 1/k, engine.py:1018-1023) looked up
            # inside the one-launch layer kernel (hsmoe_moe_layer_decode_routed)
            # a copy unless the caller owns the ids: a caller may rewrite its id
            # buffer in place (GreedyDecoder does)
            ids = input_ids.reshape(-1) if ids_owned else input_ids.reshape(-1).clone()
            ops.moe_layer_decode_routed(
                flat, tid2eid, table, SCALE_E8M0, self.store.shared_entry(layer_idx),
                self.config.moe_intermediate_size, weight_all=1.0 / k, token_ids=ids, top_k=k,
                swiglu_limit=self.config.swiglu_limit, out_f32=out_f32, out_bf16=out_bf16, norm=norm)
            self._last_routed_idx = (tid2eid, ids)
            return True
        return False

    def _forward_ffn_norm(self, hn: torch.Tensor, lw: dict, layer_idx: int, input_ids, h: torch.Tensor,
                          weight: torch.Tensor, residual: torch.Tensor | None = None, ids_owned: bool = False):
        """_forward_ffn of normed rows hn [B, T, D] followed by the next
        layer's adds and RMSNorm, in one launch: -> (h + FFN (+ residual),
        its RMSNorm) [B, T, D], bit-identical to _forward_ffn then add_rms_norm;
        None (nothing launched) where the one-launch layer does not apply."""
        B, T, D = hn.shape
        flat = hn.reshape(B * T, D)
        h2 = h.reshape(B * T, D)
        if h2.dtype != torch.bfloat16 or not h2.is_contiguous():
            return None
        norm = ops.NormTail(h2, weight, residual, self.config.rms_norm_eps)
        if not self._one_launch_layer(flat, lw, layer_idx, input_ids, norm=norm, ids_owned=ids_owned):
            return None
        return norm.h_out.reshape(B, T, D), norm.norm_out.reshape(B, T, D)

    # ------------------------------------------------------------ MTP verify
    def _snapshot_verify_state(self):
        return None

    def _restore_verify_state(self, snapshot, n_accept: int, t_total: int) -> None:
        return None

    def _final_hidden(self, h: torch.Tensor) -> torch.Tensor:
        """h [B, T, D] after the last layer -> normed hidden [B*T, D] (engine.py:2480-2482)."""
        h2 = h.reshape(-1, h.shape[-1])
        if self.norm_weight is not None:
            h2 = rms_norm(h2, self.norm_weight, self.config.rms_norm_eps)
        return h2

    # a verify whose layer kernel reports a give-up runs again on the staged
    # kernels (False: it raises HsmoeError instead)
    verify_fallback = True

    @torch.no_grad()
    def _mtp_verify_batched(self, draft_ids, temperature: float = 0.6, main_pred_id=None):
        """One fused forward of [main_pred, drafts] (engine.py:2431-2540) ->
        (n_accept, bonus_logits [1, V]); greedy acceptance on the device."""
        if not isinstance(draft_ids, torch.Tensor) or draft_ids.shape[1] == 0:
            return 0, None
        combined = torch.cat([main_pred_id, draft_ids], dim=-1) if main_pred_id is not None else draft_ids
        t_total = combined.shape[1]
        snap = self._snapshot_verify_state()
        pos_bak = self._global_pos
        n_accept = 0
        bonus_logits = None
        try:
            self._global_pos = pos_bak + 1
            self._phase = "verify"
            _, hf = self._forward_stack(combined)
            logits, pred, result = ops.lm_head_accept(hf, self.lm_head, combined.reshape(-1))
            # the one host sync per verify also reads the layer kernels' status words
            words = [w.to(torch.int64) for w in ops.moe_layer_status_words(self.device)]
            vals = torch.cat([result] + words).tolist()
            if any(vals[2:]):
                # a cross-workgroup wait of the persistent layer kernel gave up
                # (its grid was not co-resident, e.g. beside another kernel):
                # reported once, then the verify runs again on the router and
                # staged expert kernels, which need no co-residency and give
                # the same values
                ops.clear_moe_layer_status(self.device)
                if not self.verify_fallback:
                    raise ops._lib.HsmoeError(f"moe_layer_kernel: a cross-workgroup wait gave up (status "
                                              f"{max(vals[2:])}); this verify's outputs are not valid")
                warnings.warn(f"moe_layer_kernel: a cross-workgroup wait gave up (status {max(vals[2:])}); "
                              f"the verify runs again on the staged kernels", RuntimeWarning, stacklevel=2)
                self._restore_verify_state(snap, 0, t_total)
                snap = self._snapshot_verify_state()
                had = self.__dict__.get("use_one_launch_layer")
                self.use_one_launch_layer = False
                try:
                    _, hf = self._forward_stack(combined)
                finally:
                    if had is None:
                        del self.use_one_launch_layer
                    else:
                        self.use_one_launch_layer = had
                logits, pred, result = ops.lm_head_accept(hf, self.lm_head, combined.reshape(-1))
                vals = result.tolist()
            n_accept, bonus_row = vals[0], vals[1]
            bonus_logits = logits[bonus_row:bonus_row + 1]
        finally:
            self._global_pos = pos_bak + n_accept
            self._restore_verify_state(snap, n_accept, t_total)
        return n_accept, bonus_logits

    def _embed(self, ids: torch.Tensor) -> torch.Tensor:
        if self.embed is None:
            raise RuntimeError("no embedding table: pass embed= or override _embed")
        return self.embed[ids].to(torch.bfloat16)

    def _embed_fusable(self, ids: torch.Tensor) -> bool:
        """The lookup can run inside the first norm's launch (hsmoe_embed_add_rms_norm /
        hsmoe_mtp_input): this class's _embed on a bf16 [V, D] table on the ids' device."""
        e = self.embed
        return (type(self)._embed is HomeSeekMoEEngine._embed and e is not None and e.dtype == torch.bfloat16
                and e.dim() == 2 and e.is_contiguous() and e.device == ids.device and ids.dtype == torch.int64)

    # ------------------------------------------------------------ MTP draft + decode loop
    @torch.no_grad()
    def _mtp_generate_draft(self, last_hidden: torch.Tensor, num_draft: int = 2, temperature: float = 0.0,
                            last_token_id: torch.Tensor | None = None, out: torch.Tensor | None = None):
        """Greedy drafts from the MTP block (engine.py:2251-2339, stand-in described
        in the module docstring) -> (draft_ids [1, n] int64, n); no host sync.
        out (contiguous int64 [n], optional) is where the drafts are written."""
        mw = self._mtp_weights
        if mw is None or self.embed is None or self.lm_head is None or last_token_id is None or num_draft < 1:
            return None, 0
        eps = self.config.rms_norm_eps
        D = last_hidden.shape[-1]
        if out is None:
            out = torch.empty(num_draft, dtype=torch.int64, device=last_hidden.device)
        h_prev = last_hidden.reshape(1, 1, D)
        tok = last_token_id.reshape(1, 1)
        lw = mw["layer"]
        for j in range(num_draft):
            if lw.get("ffn_norm.weight") is not None and self._embed_fusable(tok):
                # embedding, enorm, hnorm, their sum, the residual add and ffn_norm in one launch
                h1, hn = ops.mtp_input(tok, self.embed, h_prev, mw["enorm.weight"], mw["hnorm.weight"],
                                       lw["ffn_norm.weight"], lw.get("attn.residual"), eps)
                h1, hn = h1.reshape(1, 1, D), hn.reshape(1, 1, D)
                fused = self._forward_ffn_norm(hn, lw, mw["layer_idx"], tok, h1, mw["norm.weight"], ids_owned=True)
                if fused is not None:
                    h_prev, hf = fused[0], fused[1].reshape(-1, D)
                else:
                    ffn_out, _ = self._forward_ffn(hn, lw, mw["layer_idx"], tok)
                    h_prev = h1 + ffn_out
                    hf = rms_norm(h_prev.reshape(-1, D), mw["norm.weight"], eps)
            else:
                e = rms_norm(self._embed(tok).reshape(1, D), mw["enorm.weight"], eps)
                h_in = rms_norm(h_prev.reshape(1, D), mw["hnorm.weight"], eps) + e
                h_prev, hf = self._forward_layer_norm(h_in.reshape(1, 1, D), lw, mw["layer_idx"], tok,
                                                      mw["norm.weight"])
            ops.lm_head_accept(hf, self.lm_head, None, want_logits=False, pred=out[j:j + 1])
            tok = out[j:j + 1].reshape(1, 1)
        return out[:num_draft].reshape(1, num_draft), num_draft

    def _next_norm(self, layer_idx: int, final_norm: bool):
        """(residual, norm weight) that follow layer layer_idx's FFN: the next
        layer's attention stand-in and ffn_norm, or after the last layer the
        final norm (no residual); None when no fused norm follows."""
        if layer_idx + 1 < self.config.num_hidden_layers:
            lw = self._get_layer_weights(layer_idx + 1)
            w = lw.get("ffn_norm.weight")
            return None if w is None else (lw.get("attn.residual"), w)
        if final_norm and self.norm_weight is not None:
            return None, self.norm_weight
        return None

    def _forward_stack(self, ids: torch.Tensor, final_norm: bool = True):
        """Embed ids [1, T] and run every layer -> (last hidden [1, T, D], its
        final RMSNorm [T, D] or None).  Same values as _forward_layer in a loop:
        where the one-launch layer applies, each layer launch ends with the
        next layer's residual adds and RMSNorm (or the final norm); elsewhere
        the FFN output is added in the next add + norm launch
        (hsmoe_add_rms_norm), which also adds that layer's residual."""
        eps = self.config.rms_norm_eps
        n_layers = self.config.num_hidden_layers
        hn = None  # this layer's normed input, when the previous launch made it
        pending = None  # FFN output of the previous layer, not yet added
        lw0 = self._get_layer_weights(0) if n_layers > 0 else {}
        if lw0.get("ffn_norm.weight") is not None and self._embed_fusable(ids):
            # lookup + first layer's residual add + RMSNorm in one launch
            h, hn = ops.embed_add_rms_norm(ids, self.embed, lw0["ffn_norm.weight"], lw0.get("attn.residual"), eps)
        else:
            h = self._embed(ids)
        for layer_idx in range(n_layers):
            lw = self._get_layer_weights(layer_idx)
            norm_w = lw.get("ffn_norm.weight")
            # a hash layer keeps a private copy of the ids only when it is the
            # last layer: otherwise a later layer replaces _last_routed_idx
            # before this call returns
            ids_owned = layer_idx + 1 < n_layers
            if norm_w is None:
                if pending is not None:
                    h, pending = h + pending, None
                h, _ = self._forward_layer(h, lw, layer_idx, ids)
                continue
            if hn is None:
                h, hn = ops.add_rms_norm(h, norm_w, add=pending, residual=lw.get("attn.residual"), eps=eps,
                                         want_sum=True)
                pending = None
            nxt = self._next_norm(layer_idx, final_norm)
            fused = None if nxt is None else self._forward_ffn_norm(hn, lw, layer_idx, ids, h, nxt[1], nxt[0],
                                                                    ids_owned=ids_owned)
            if fused is not None:
                h, hn = fused
                continue
            pending, _ = self._forward_ffn(hn, lw, layer_idx, ids)
            hn = None
        if final_norm and self.norm_weight is not None:
            if hn is not None:  # the last layer's launch made the final norm
                return h, hn.reshape(-1, h.shape[-1])
            h, hf = ops.add_rms_norm(h, self.norm_weight, add=pending, eps=eps, want_sum=True)
            return h, hf.reshape(-1, h.shape[-1])
        if pending is not None:
            h = h + pending
        return h, (self._final_hidden(h) if final_norm else None)

    def draft_count(self) -> int:
        """Drafts per decode step: config.mtp_num_draft when the MTP block, the
        embedding and lm_head are present, else 0 (plain greedy decode)."""
        has_mtp = self._mtp_weights is not None and self.embed is not None and self.lm_head is not None
        return max(0, int(self.config.mtp_num_draft)) if has_mtp else 0

    @torch.no_grad()
    def decode_step(self, cur: torch.Tensor, out_row: torch.Tensor | None = None, record: tuple | None = None,
                    cur_out: torch.Tensor | None = None):
        """One greedy decode step, on the device only (engine.py:2809-2922 at
        temperature 0): M=1 forward of `cur` -> main token A; with n_draft =
        draft_count() > 0, drafts [d_0 .. d_{n_draft-1}] from the MTP block and
        one verify of [A, drafts]; n = accepted drafts.  Returns (row
        [2 + n_draft] = A, drafts, bonus token (row [1] = A without drafts);
        count of tokens emitted = 1 + (n > 0) * (n + 1); next token to forward
        (the bonus when n > 0, else A, which the next step forwards as the
        reference's loop does); n), all device tensors.  record = (rows, counts,
        n_accepts, k) also stores the step as row k (advancing k on the device)
        and cur_out receives the next token, in the step's last launch."""
        cur = cur.reshape(1, 1)
        n_draft = self.draft_count()
        toks = torch.empty(1 + n_draft, dtype=torch.int64, device=cur.device)  # [A, drafts]: the verify's ids
        h, hf = self._forward_stack(cur)
        ops.lm_head_accept(hf, self.lm_head, None, want_logits=False, pred=toks[:1])
        drafts = None
        if n_draft > 0:
            own = (type(self)._mtp_generate_draft is HomeSeekMoEEngine._mtp_generate_draft
                   and "_mtp_generate_draft" not in self.__dict__)
            if own:  # the drafts go straight into the verify's id buffer
                drafts, n_draft = self._mtp_generate_draft(h, n_draft, 0.0, last_token_id=toks[:1], out=toks[1:])
            else:  # an override with the reference's signature
                drafts, n_draft = self._mtp_generate_draft(h, n_draft, 0.0, last_token_id=toks[:1])
                if drafts is not None and n_draft > 0:
                    toks = torch.cat([toks[:1], drafts.reshape(-1)[:n_draft].to(torch.int64)])
        if drafts is None or n_draft == 0:
            row, count, nxt, n_acc = ops.decode_step_record(toks[:1], record=record, cur=cur_out)
        else:
            toks = toks[:1 + n_draft]
            _, hfv = self._forward_stack(toks.reshape(1, -1))
            _, pred_v, result = ops.lm_head_accept(hfv, self.lm_head, toks, want_logits=False)
            row, count, nxt, n_acc = ops.decode_step_record(toks, pred_v, result, record=record, cur=cur_out)
        if out_row is not None:
            out_row.copy_(row)
        return row, count, nxt, n_acc

    @torch.no_grad()
    def generate_greedy(self, first_id: int, steps: int, graph: bool = True):
        """`steps` decode steps from token first_id -> (tokens list, accepted
        drafts per step).  With graph=True one step is captured as a HIP graph
        and replayed: no host synchronisation until the end."""
        dec = GreedyDecoder(self, steps, graph)
        dec.reset(first_id)
        dec.run(steps)
        return dec.result()

    # ------------------------------------------------------------ layer stand-in
    def _forward_layer(self, h: torch.Tensor, lw: dict, layer_idx: int, input_ids=None):
        """Layer with attention replaced by a fixed residual lw["attn.residual"] [D]:
        h = h + r; h = h + FFN(rms_norm(h, ffn_norm))  (engine.py:2653-2690 without mHC)."""
        r = lw.get("attn.residual")
        norm_w = lw.get("ffn_norm.weight")
        if norm_w is not None:
            h, hn = ops.add_rms_norm(h, norm_w, residual=r, eps=self.config.rms_norm_eps, want_sum=True)
        else:
            if r is not None:
                h = h + r
            hn = h
        ffn_out, used = self._forward_ffn(hn, lw, layer_idx, input_ids)
        return h + ffn_out, used

    def _forward_layer_norm(self, h: torch.Tensor, lw: dict, layer_idx: int, input_ids, weight: torch.Tensor):
        """_forward_layer followed by an RMSNorm with `weight` -> (h [B, T, D],
        normed [B*T, D]); the norm runs in the layer's launch where the
        one-launch layer applies (same values)."""
        norm_w = lw.get("ffn_norm.weight")
        if norm_w is not None:
            h1, hn = ops.add_rms_norm(h, norm_w, residual=lw.get("attn.residual"), eps=self.config.rms_norm_eps,
                                      want_sum=True)
            fused = self._forward_ffn_norm(hn, lw, layer_idx, input_ids, h1, weight)
            if fused is not None:
                return fused[0], fused[1].reshape(-1, h.shape[-1])
            ffn_out, _ = self._forward_ffn(hn, lw, layer_idx, input_ids)
            h_out = h1 + ffn_out
        else:
            h_out, _ = self._forward_layer(h, lw, layer_idx, input_ids)
        return h_out, rms_norm(h_out.reshape(-1, h.shape[-1]), weight, self.config.rms_norm_eps)


class GreedyDecoder:
    """Device-resident greedy decode loop with MTP verify (engine.py:2809-2922 at
    temperature 0).  Per step it records the row [A, drafts, bonus], the count of
    tokens emitted and the accepted drafts into device buffers of `capacity`
    steps, and carries the next token on the device; with graph=True one step
    is captured as a HIP graph (after one eager warm-up step, so that every
    workspace exists before capture) and replayed."""

    def __init__(self, engine: HomeSeekMoEEngine, capacity: int, graph: bool = True):
        dev = engine.device
        if capacity < 1:
            raise ValueError("a decoder needs room for at least one step")
        self.engine, self.capacity = engine, int(capacity)
        self.width = 2 + engine.draft_count() if engine.draft_count() > 0 else 1  # A, drafts, bonus
        self.rows = torch.zeros(self.capacity, self.width, dtype=torch.int64, device=dev)
        self.counts = torch.zeros(self.capacity, dtype=torch.int64, device=dev)
        self.n_accs = torch.zeros(self.capacity, dtype=torch.int64, device=dev)
        self.cur = torch.zeros(1, 1, dtype=torch.int64, device=dev)
        self.k = torch.zeros((), dtype=torch.int64, device=dev)  # next row, on the device
        self.done = 0  # rows written, on the host (bounds every run)
        self.graph = None
        if graph:
            stream = torch.cuda.Stream(device=dev)
            stream.wait_stream(torch.cuda.current_stream(dev))
            with torch.cuda.stream(stream):
                self._body()  # warm-up step into row 0, overwritten after reset()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=stream):
                    self._body()
            torch.cuda.current_stream(dev).wait_stream(stream)
            self.graph = g

    def _body(self):
        # the step's last launch (hsmoe_decode_step_record) writes row k, advances k and sets cur
        self.engine.decode_step(self.cur, record=(self.rows, self.counts, self.n_accs, self.k), cur_out=self.cur)

    def reset(self, first_id: int | None = None) -> None:
        """Rewinds the row index; first_id (if given) becomes the token to forward."""
        if first_id is not None:
            self.cur.fill_(int(first_id))
        self.k.zero_()
        self.done = 0

    def run(self, n: int) -> None:
        if self.done + n > self.capacity:
            raise ValueError(f"{n} more steps exceed the decoder's capacity of {self.capacity} rows")
        for _ in range(n):
            if self.graph is not None:
                self.graph.replay()
            else:
                self._body()
        self.done += n

    def result(self):
        """(tokens emitted, accepted drafts per step) of the rows written since
        reset().  Raises HsmoeError when a layer launch of the run reported a
        cross-workgroup wait that gave up (its outputs are not valid)."""
        ops.check_moe_layer_status(self.engine.device)
        n = self.done
        rows_h, counts_h = self.rows[:n].cpu().tolist(), self.counts[:n].cpu().tolist()
        tokens = []
        for r, c in zip(rows_h, counts_h):
            tokens.append(r[0])
            if c > 1:
                tokens.extend(r[1:c - 1] + [r[-1]])
        return tokens, self.n_accs[:n].cpu().tolist()


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """utils.py:6-9 on the HIP kernel: fp32 mean of squares, x*rsqrt(var+eps)*w, cast back."""
    return ops.rms_norm(x, weight, eps)
