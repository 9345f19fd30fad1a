"""MI355X (gfx950) paged attention: drop-in for gb10-attn's decode v1/v2/v3
and WMMA-prefill launchers, plus the KV-cache write that fills the paged pool.

The C-ABI lives in include/pagedattn.h and libpagedattn.so (built from
csrc/ by build.py); this package is its torch-facing mirror.  Import name:
gb10_attn_amd (the directory is gb10-attn_amd; __graft_entry__.load_package()
registers it).
"""
from ._lib import EXPORTS, LIB_PATH, PaTensor, check, last_error, last_launch, lib  # noqa: F401
from .ops import (choose_num_splits, choose_num_splits_for, paged_attention,  # noqa: F401
                  paged_attention_prefill, paged_attention_prefill_varlen, paged_attention_prefill_wmma,
                  paged_attention_v2,
                  paged_attention_v3, plan_partitions, torch_ops, view, workspace_size, write_kv,
                  write_kv_blocks)

__all__ = [
    "paged_attention", "paged_attention_v2", "paged_attention_v3", "choose_num_splits",
    "paged_attention_prefill", "paged_attention_prefill_wmma", "paged_attention_prefill_varlen",
    "choose_num_splits_for",
    "plan_partitions", "workspace_size", "view", "lib", "LIB_PATH", "EXPORTS", "write_kv",
    "write_kv_blocks", "torch_ops",
]
