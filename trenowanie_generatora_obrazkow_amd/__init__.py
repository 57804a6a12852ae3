"""MI355X-native (gfx950) mixture-of-experts SwiGLU layer: hand-written HIP kernels behind a C ABI
(include/hmoe.h, built as _lib/libhmoe.so), with the reference's Python call surfaces on top:

  moe_triton  -- BLOCK_M, m_bucket, make_schedule, grouped_mm   (aurora/moe_triton.py)
  hf_compat   -- fuse_moe / _fused_moe_infer (mode "hip")        (aurora/hf_compat.py:62-169)
  layer       -- MoESwiGLU, a trainable drop-in for DenoiserBlock.mlp (aurora/model.py:102-110, 201, 210)
  poziomka    -- PoziomkaMoE / PoziomkaMLP / PoziomkaGate, the BailingMoeV2 block with int8 experts and the
                 sigmoid, group-limited router (aurora/hf_pipeline.py:314-370)
  ops         -- tensor-level wrappers of every C entry point
"""
from . import _lib  # noqa: F401
from .layer import MoESwiGLU, moe_param_groups, moe_swiglu  # noqa: F401

__all__ = ["MoESwiGLU", "moe_swiglu", "moe_param_groups"]
