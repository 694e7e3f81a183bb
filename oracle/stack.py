"""CPU oracle of the synthetic MoE-only decode stack -- TEST INFRASTRUCTURE ONLY.

Restates, with the oracle's pinned pieces (router, moe_layer_fp32, rms_norm,
logits_bf16, mtp_accept), the greedy decode loop with MTP verify of the
reference engine with attention replaced by a fixed per-layer residual:
  layer        h = h + r; h = h + FFN(rms_norm(h, ffn_norm))   engine.py:2653-2690 (no mHC)
  hash routing ids = tid2eid[token], weight 1/k                 engine.py:1018-1023
  router       sqrt(softplus) + bias top-k                      router.py:22-36
  verify       [A, d0, d1] through every layer, lm_head,
               longest-prefix acceptance + bonus                engine.py:2431-2540
  MTP drafts   hnorm(h) + enorm(embed(tok)) -> MTP MoE block ->
               norm -> lm_head argmax, second draft from the
               first (no attention, no e_proj / h_proj)          engine.py:2251-2339
  decode loop  temperature 0                                     engine.py:2809-2922
The synthetic weights are regenerated with the same counter-based generators
as the device (seeded tags), the embedding is tied to lm_head, and hash layers
route token v to (b(v) + j * 41) mod E.

bf16 tensors are uint16 arrays of raw bits; a bf16 + bf16 sum is the fp32 sum
rounded once (torch's bf16 add).  The MoE FFN is fp32-accumulated and rounded
to bf16 once, which the device matches within the FFN tolerance, not bit for
bit: per-layer comparisons use that tolerance, and token streams agree where
the argmax margins exceed the propagated error.  The pieces are pinned
individually; the decode loop's emission rule (decode_step + generate) is
pinned against a direct restatement of the reference loop (engine.py:2809-2922
at temperature 0) on a toy model whose next token is known, for 0-3 drafts.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as orc

HASH_STEP = 41


def bf16_add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return orc.f32_to_bf16((orc.bf16_to_f32(a) + orc.bf16_to_f32(b)).astype(np.float32))


class StackOracle:
    """The synthetic stack of seed `seed` at any size (store layer n_layers = MTP block)."""

    def __init__(self, seed: int, n_layers: int, n_experts: int, d: int, i: int, vocab: int, top_k: int = 6,
                 n_hash: int = 3, scaling: float = 1.5, limit: float = 10.0, eps: float = 1e-6,
                 cache: bool = True, workers: int = 0):
        """cache=False regenerates experts on every use (host memory stays at
        the few experts in flight: a full-size stack holds 11,008 of them);
        workers > 0 evaluates a layer's experts and logits rows on that many
        threads (the C generators and numpy release the GIL), with results
        equal to the serial ones bit for bit."""
        self.seed, self.n_layers, self.E, self.d, self.i = seed, n_layers, n_experts, d, i
        self.vocab, self.k, self.n_hash = vocab, top_k, n_hash
        self.scaling, self.limit, self.eps = scaling, limit, eps
        self.cache = cache
        self._pool = None
        if workers > 0:
            from concurrent.futures import ThreadPoolExecutor
            self._pool = ThreadPoolExecutor(max_workers=workers)
        self._experts: dict = {}
        self._shared: dict = {}
        self.layers = [self._layer_weights(l, hashed=l < n_hash) for l in range(n_layers)]
        self.lm_head = self._normal(orc.tag(orc.KIND_LM_HEAD), vocab * d, 0.0, 0.02).reshape(vocab, d)
        self.final_norm = self._normal(orc.tag(orc.KIND_NORM_W, 0xFFFF), d, 1.0, 0.05)
        self.mtp = {
            "layer": self._layer_weights(n_layers, hashed=False),
            "layer_idx": n_layers,
            "hnorm": self._normal(orc.tag(orc.KIND_NORM_W, 0xFFFF, 1), d, 1.0, 0.05),
            "enorm": self._normal(orc.tag(orc.KIND_NORM_W, 0xFFFF, 2), d, 1.0, 0.05),
            "norm": self._normal(orc.tag(orc.KIND_NORM_W, 0xFFFF, 3), d, 1.0, 0.05),
        }

    # ------------------------------------------------------------ weights
    def _normal(self, t: int, n: int, mean: float, std: float) -> np.ndarray:
        return orc.gen_normal_bf16(orc.key(self.seed, t), n, mean, std)

    def _layer_weights(self, layer: int, hashed: bool) -> dict:
        d, E = self.d, self.E
        lw = {
            "gate": self._normal(orc.tag(orc.KIND_GATE_W, layer), E * d, 0.0, 0.02).reshape(E, d),
            "bias": orc.gen_normal_f32(orc.key(self.seed, orc.tag(orc.KIND_GATE_BIAS, layer)), E, 0.0, 0.01),
            "ffn_norm": self._normal(orc.tag(orc.KIND_NORM_W, layer), d, 1.0, 0.05),
            "residual": self._normal(orc.tag(orc.KIND_RESIDUAL, layer), d, 0.0, 0.1),
        }
        if hashed:
            base = orc.gen_index(orc.key(self.seed, orc.tag(orc.KIND_TID2EID, layer)), self.vocab, E)
            lw["tid2eid"] = (base[:, None] + np.arange(self.k, dtype=np.int64)[None, :] * HASH_STEP) % E
        return lw

    def expert(self, layer: int, eid: int) -> dict:
        if not self.cache:
            return orc.gen_fp4_expert(self.seed, layer, eid, self.d, self.i)
        if (layer, eid) not in self._experts:
            self._experts[(layer, eid)] = orc.gen_fp4_expert(self.seed, layer, eid, self.d, self.i)
        return self._experts[(layer, eid)]

    def shared(self, layer: int) -> dict:
        if not self.cache:
            return orc.gen_shared_expert(self.seed, layer, self.d, self.i)
        if layer not in self._shared:
            self._shared[layer] = orc.gen_shared_expert(self.seed, layer, self.d, self.i)
        return self._shared[layer]

    # ------------------------------------------------------------ one layer
    def route(self, hn: np.ndarray, lw: dict, ids: np.ndarray | None):
        """-> (idx [T, k] int64, w [T, k] fp32); hash layers use the token table."""
        if "tid2eid" in lw and ids is not None:
            idx = lw["tid2eid"][np.asarray(ids, dtype=np.int64).reshape(-1)]
            return idx, np.full(idx.shape, np.float32(1.0 / self.k), dtype=np.float32)
        return orc.router(hn, lw["gate"], lw["bias"], self.k, self.scaling)

    def ffn(self, hn: np.ndarray, lw: dict, layer: int, ids) -> tuple[np.ndarray, np.ndarray]:
        """Routed + shared FFN of normed hidden hn [T, D] -> (fp32 out [T, D], idx)."""
        idx, w = self.route(hn, lw, ids)
        if self.cache and self._pool is None:
            experts = {int(e): self.expert(layer, int(e)) for e in np.unique(idx)}
            return orc.moe_layer_fp32(hn, idx, w, experts, self.shared(layer), self.limit), idx
        return orc.moe_layer_fp32_lazy(hn, idx, w, lambda e: self.expert(layer, e), lambda: self.shared(layer),
                                       self.limit, self._pool), idx

    def layer(self, h: np.ndarray, lw: dict, layer: int, ids) -> dict:
        """One layer on bf16 h [T, D] -> {"h1": h + r, "hn": normed, "ffn": fp32, "idx", "out": bf16}."""
        h1 = bf16_add(h, lw["residual"][None, :])
        hn = orc.rms_norm(h1, lw["ffn_norm"], self.eps)
        f, idx = self.ffn(hn, lw, layer, ids)
        return {"h1": h1, "hn": hn, "ffn": f, "idx": idx, "out": bf16_add(h1, orc.f32_to_bf16(f))}

    # ------------------------------------------------------------ stack, head, MTP
    def embed(self, ids) -> np.ndarray:
        return self.lm_head[np.asarray(ids, dtype=np.int64).reshape(-1)]

    def forward_stack(self, ids) -> np.ndarray:
        h = self.embed(ids)
        for l in range(self.n_layers):
            h = self.layer(h, self.layers[l], l, ids)["out"]
        return h

    def logits(self, h: np.ndarray, norm_w: np.ndarray) -> np.ndarray:
        hn = orc.rms_norm(h, norm_w, self.eps)
        if self._pool is None or hn.shape[0] == 1:
            return orc.logits_bf16(hn, self.lm_head)
        rows = list(self._pool.map(lambda t: orc.logits_bf16(hn[t:t + 1], self.lm_head), range(hn.shape[0])))
        return np.concatenate(rows, axis=0)

    def argmax(self, logits: np.ndarray) -> list[int]:
        return [orc.argmax_first(logits[t]) for t in range(logits.shape[0])]

    def drafts(self, h_last: np.ndarray, tok: int, n: int = 2, margins: list | None = None) -> list[int]:
        mw = self.mtp
        h_prev, out = h_last.reshape(1, self.d), []
        for _ in range(n):
            e = orc.rms_norm(self.embed([tok]), mw["enorm"], self.eps)
            h_in = bf16_add(orc.rms_norm(h_prev, mw["hnorm"], self.eps), e)
            h_prev = self.layer(h_in, mw["layer"], mw["layer_idx"], [tok])["out"]
            lg = self.logits(h_prev, mw["norm"])
            if margins is not None:
                margins.append(top2_gap(lg[0]))
            tok = self.argmax(lg)[0]
            out.append(tok)
        return out

    def next_token(self, tok: int) -> int:
        """Greedy M=1 decode of one token (no attention: the next token is a function of this one)."""
        return self.argmax(self.logits(self.forward_stack([tok]), self.final_norm))[0]

    def decode_step(self, cur: int, margins: list | None = None, draft_fn=None, n_draft: int = 2):
        """-> (row [A, drafts, bonus] ([A] without drafts), count, next token,
        n_accept); draft_fn(h, A) replaces the MTP block's drafts when given;
        n_draft = 0 is the reference's plain greedy step (engine.py:2858-2862)."""
        h = self.forward_stack([cur])
        lg = self.logits(h, self.final_norm)
        a = self.argmax(lg)[0]
        if margins is not None:
            margins.append(top2_gap(lg[0]))
        if n_draft == 0 and draft_fn is None:
            return [a], 1, a, 0
        dr = self.drafts(h, a, n_draft, margins) if draft_fn is None else list(draft_fn(h, a))
        combined = [a] + dr
        lv = self.logits(self.forward_stack(combined), self.final_norm)
        if margins is not None:
            margins.extend(top2_gap(lv[t]) for t in range(lv.shape[0]))
        n_acc, bonus_row = orc.mtp_accept(lv, combined)
        bonus = self.argmax(lv[bonus_row:bonus_row + 1])[0]
        count = 1 + (n_acc + 1 if n_acc > 0 else 0)
        return [a] + dr + [bonus], count, (bonus if n_acc > 0 else a), n_acc

    def generate(self, first: int, steps: int, margins: list | None = None, draft_fn=None, n_draft: int = 2):
        """Greedy decode -> (tokens, accepted drafts per step), as the device loop emits them."""
        cur, tokens, accs = first, [], []
        for _ in range(steps):
            row, count, cur, n_acc = self.decode_step(cur, margins, draft_fn, n_draft)
            tokens.append(row[0])
            if count > 1:
                tokens.extend(row[1:count - 1] + [row[-1]])
            accs.append(n_acc)
        return tokens, accs


def top2_gap(row_bf16: np.ndarray) -> float:
    v = np.sort(orc.bf16_to_f32(row_bf16).astype(np.float64))
    return float(v[-1] - v[-2])
