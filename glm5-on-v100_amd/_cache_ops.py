"""Drop-in for vLLM's MLA cache writer (vllm/_custom_ops.py
concat_and_cache_mla), the producer of the latent cache the sparse MLA
kernels read: same name, argument order and semantics for kv_cache_dtype
"auto" and "fp8_ds_mla".  It dispatches to the torch op registered by
ops.py, which runs the gfx950 HIP kernel.
"""
from __future__ import annotations

import torch

from ._sm70_ops import _op


def concat_and_cache_mla(kv_c: torch.Tensor, k_pe: torch.Tensor, kv_cache: torch.Tensor,
                         slot_mapping: torch.Tensor, kv_cache_dtype: str,
                         scale: torch.Tensor) -> None:
    """Writes token t of kv_c [T, 512] and k_pe [T, 64] into the latent cache
    row slot_mapping[t] (T = slot_mapping.numel(); negative slots skipped).

    "auto": kv_cache fp16 [n_blocks, page, 576] = [kv_c | k_pe].
    "fp8_ds_mla": kv_cache uint8 [n_blocks, page, 656]: 512 e4m3 bytes with a
    max(amax/448, FLT_MIN) scale per 128-dim tile, the 4 fp32 scales, then the
    64 16-bit RoPE values.  `scale` is unused by both (vLLM reads it only for
    per-tensor fp8 caches)."""
    _op("concat_and_cache_mla")(kv_c, k_pe, kv_cache, slot_mapping, kv_cache_dtype, scale)
