"""MI355X (gfx950) routed-expert MoE hot path of Home-Seek.

Imported as `home_seek_amd` (the directory name carries a hyphen; see
__graft_entry__.package()).  Modules mirror the reference's operator API:
  fused_moe      FusedMoEFFN, SharedExpertFFN, fused_expert_ffn_*, dequant
  router         compute_expert_affinity(_with_bias), stable_topk
  _fp4           unpack_from_e2m1fn_x2, transform_sf, cast_back
  engine         HomeSeekMoEEngine: loaders, _forward_ffn, _mtp_verify_batched
  expert_store   HbmExpertStore: all experts resident in HBM
  ops            thin torch wrappers over the C ABI (include/hsmoe.h)
The compute runs in libhsmoe.so (csrc/, hand-written HIP for gfx950); there is
no CPU or Triton fallback.
"""
from ._lib import HsmoeError, LIB_PATH, lib  # noqa: F401

__version__ = "0.1.0"
