"""HBM-resident expert store: every routed FP4 expert of every layer, plus the
FP8 shared experts, in one device allocation.

Replaces the reference's four expert tiers -- GPU hot FIFO, GPU BF16 FIFO,
CPU pinned FP4 LRU and disk mmap (engine.py:185-191, expert_cache.py:7-116,
engine.py:1054-1335) -- because 43 x 256 experts of 13,369,344 bytes
(147.2 GB) fit in one MI355X's 288 GB.  Experts keep the checkpoint's layout
(safetensors keys layers.{L}.ffn.experts.{E}.w{1,3,2}.{weight,scale}):
  w1, w3  int8 [I, D/2]   packed e2m1, low nibble = even column
  w2      int8 [D, I/2]
  scales  float8_e8m0fnu [I, D/32], [D, I/32]
so loader calls return views, never copies.  One expert record is
[w1 | w3 | w2 | s1 | s3 | s2], 256-byte aligned.  The FP8 shared experts
(e4m3 [I, D], [I, D], [D, I] + fp32 128x128 block scales) follow the routed
region.
"""
from __future__ import annotations

import torch

from . import ops, synthetic


def _align(n: int, a: int = 256) -> int:
    return (n + a - 1) // a * a


class HbmExpertStore:
    def __init__(self, n_layers: int, n_experts: int = 256, hidden_size: int = 4096,
                 intermediate_size: int = 2048, device: str | torch.device = "cuda",
                 with_shared: bool = True):
        self.n_layers = n_layers
        self.n_experts = n_experts
        self.d = d = hidden_size
        self.i = i = intermediate_size
        self.device = torch.device(device)
        if d % 128 or i % 128:
            raise ValueError("hidden and intermediate sizes must be multiples of 128")
        # byte offsets inside one routed-expert record
        self._shape = {
            "w1": (i, d // 2), "w3": (i, d // 2), "w2": (d, i // 2),
            "s1": (i, d // 32), "s3": (i, d // 32), "s2": (d, i // 32),
        }
        off = 0
        self._off = {}
        for name in ("w1", "w3", "w2", "s1", "s3", "s2"):
            self._off[name] = off
            r, c = self._shape[name]
            off = _align(off + r * c)
        self.expert_bytes = off
        self.payload_bytes = 3 * i * d // 2 + 3 * i * d // 32  # 13,369,344 at D=4096, I=2048
        # shared FP8 expert record
        sh = {"w1": (i, d, 1), "w3": (i, d, 1), "w2": (d, i, 1),
              "s1": (i // 128, d // 128, 4), "s3": (i // 128, d // 128, 4), "s2": (d // 128, i // 128, 4)}
        soff = 0
        self._soff = {}
        self._sshape = sh
        for name in ("w1", "w3", "w2", "s1", "s3", "s2"):
            self._soff[name] = soff
            r, c, es = sh[name]
            soff = _align(soff + r * c * es)
        self.shared_bytes = soff if with_shared else 0
        self.with_shared = with_shared
        self.routed_region = n_layers * n_experts * self.expert_bytes
        total = self.routed_region + n_layers * self.shared_bytes
        self.buf = torch.empty(total, dtype=torch.uint8, device=self.device)
        self._tables: dict[int, torch.Tensor] = {}
        self._shared_entries: dict[int, torch.Tensor] = {}
        self._absent: set[tuple[int, int]] = set()  # experts a checkpoint does not hold
        self._no_shared: set[int] = set()           # layers without a shared expert

    # ------------------------------------------------------------ presence
    def mark_absent(self, layer: int, eid: int) -> None:
        """The expert is not in the checkpoint: its table row becomes zero (the
        kernels skip it, as the reference skips a loader returning None)."""
        self._expert_base(layer, eid)
        self._absent.add((layer, eid))
        self._tables.pop(layer, None)

    def has_expert(self, layer: int, eid: int) -> bool:
        return 0 <= layer < self.n_layers and 0 <= eid < self.n_experts and (layer, eid) not in self._absent

    def mark_no_shared(self, layer: int) -> None:
        self._no_shared.add(layer)
        self._shared_entries.pop(layer, None)

    def has_shared(self, layer: int) -> bool:
        return self.with_shared and layer not in self._no_shared

    # ------------------------------------------------------------ views
    def _expert_base(self, layer: int, eid: int) -> int:
        if not (0 <= layer < self.n_layers and 0 <= eid < self.n_experts):
            raise IndexError(f"expert ({layer}, {eid}) outside the store")
        return (layer * self.n_experts + eid) * self.expert_bytes

    def expert_views(self, layer: int, eid: int):
        """(w1, w1_scale, w3, w3_scale, w2, w2_scale) views: int8 data, E8M0 scales."""
        base = self._expert_base(layer, eid)
        out = []
        for name in ("w1", "s1", "w3", "s3", "w2", "s2"):
            r, c = self._shape[name]
            t = self.buf[base + self._off[name]: base + self._off[name] + r * c].view(r, c)
            out.append(t.view(torch.int8) if name.startswith("w") else t.view(torch.float8_e8m0fnu))
        return tuple(out)

    def shared_views(self, layer: int):
        """(w1, s1, w3, s3, w2, s2): e4m3 data and fp32 block scales of the shared expert."""
        if not self.with_shared:
            return None
        base = self.routed_region + layer * self.shared_bytes
        out = []
        for name in ("w1", "s1", "w3", "s3", "w2", "s2"):
            r, c, es = self._sshape[name]
            t = self.buf[base + self._soff[name]: base + self._soff[name] + r * c * es]
            out.append(t.view(torch.float8_e4m3fn).view(r, c) if es == 1 else t.view(torch.float32).view(r, c))
        return tuple(out)

    def table(self, layer: int) -> torch.Tensor:
        """Device uint64 [n_experts, 6] address table of a layer (cached)."""
        t = self._tables.get(layer)
        if t is None:
            base = self.buf.data_ptr() + layer * self.n_experts * self.expert_bytes
            rows = []
            for e in range(self.n_experts):
                b = base + e * self.expert_bytes
                if (layer, e) in self._absent:
                    rows.append([0] * 6)
                else:
                    rows.append([b + self._off[n] for n in ("w1", "s1", "w3", "s3", "w2", "s2")])
            t = torch.tensor(rows, dtype=torch.int64).to(self.device)
            self._tables[layer] = t
        return t

    def shared_entry(self, layer: int) -> torch.Tensor | None:
        if not self.has_shared(layer):
            return None
        t = self._shared_entries.get(layer)
        if t is None:
            t = ops.shared_entry(*self.shared_views(layer), device=self.device)
            self._shared_entries[layer] = t
        return t

    # ------------------------------------------------------------ integrity
    def expert_record(self, layer: int, eid: int) -> torch.Tensor:
        """uint8 view of one routed expert's record [w1 | w3 | w2 | s1 | s3 | s2]."""
        base = self._expert_base(layer, eid)
        return self.buf[base: base + self.expert_bytes]

    def layer_region(self, layer: int) -> torch.Tensor:
        """uint8 view of one layer's routed experts (n_experts records)."""
        if not 0 <= layer < self.n_layers:
            raise IndexError(f"layer {layer} outside the store")
        base = layer * self.n_experts * self.expert_bytes
        return self.buf[base: base + self.n_experts * self.expert_bytes]

    def checksum(self, region: torch.Tensor | None = None) -> torch.Tensor:
        """XOR of the 16-byte words of `region` (a view of this store, e.g.
        layer_region(l) or expert_record(l, e)), or of the whole store: uint8
        [16] on the device (hsmoe_xor_checksum), to compare with a checksum of
        the source bytes after a load."""
        return ops.xor_checksum(self.buf if region is None else region)

    # ------------------------------------------------------------ fill
    def fill_synthetic(self, seed: int, layers=None) -> None:
        """Fills experts (and shared experts) with the seeded synthetic weights."""
        for layer in (range(self.n_layers) if layers is None else layers):
            for eid in range(self.n_experts):
                synthetic.fill_fp4_expert(seed, layer, eid, self.expert_views(layer, eid))
            if self.with_shared:
                synthetic.fill_shared_expert(seed, layer, self.shared_views(layer))
