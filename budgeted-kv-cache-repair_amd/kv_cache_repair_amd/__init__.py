"""MI355X-native packed refresh executor for budgeted KV-cache repair.

Drop-in for the packed path of yh0903/budgeted-kv-cache-repair on AMD gfx950:
RoPE delta rotation, indexed K/V scatter and packed causal attention run as
hand-written HIP kernels in ``libkvrepair.so`` (C ABI in include/kvrepair.h).
"""

from .api import RepairResult, Selection, repair_after_deletion, repair_with_positions, select_support

__all__ = ["RepairResult", "Selection", "repair_after_deletion", "repair_with_positions", "select_support"]
