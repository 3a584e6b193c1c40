"""kvpath: Kelpie's paged-KV hot path (append, gather, paged attention, copy_blocks) as
hand-written HIP kernels for MI355X (gfx950) behind a C ABI (include/kvpath.h).

    import kvpath
    out = torch.ops.kvpath.paged_attention(q, k, v, kv_member, row_request, positions,
                                           query_start_loc, seq_lens, block_table,
                                           slot_mapping, window, sinks, causal)

The op's signature, layout and plan contract are kelpie's `kelpie::paged_attention`
(kelpie/kelpie-models/kelpie_models/kernels/ops/paged_attention.py:67-140);
`kvpath.kelpie_adapter.register()` plugs it into kelpie's op registry as impl "mi355x".
"""

from kvpath.paged_attention import (
    KV_MEMBERS,
    assert_newest_positions,
    attend,
    check_plan_status,
    clear_plan_status,
    copy_blocks,
    kv_gather,
    kv_views,
    new_kv_scale,
    no_sinks,
    paged_attention,
    paged_attention_fp8,
    plan_status,
    set_slot_check,
    split_plan,
    workspace_bytes,
    workspace_bytes_max,
    write_kv,
)

__all__ = [
    "KV_MEMBERS",
    "assert_newest_positions",
    "attend",
    "check_plan_status",
    "clear_plan_status",
    "copy_blocks",
    "kv_gather",
    "kv_views",
    "new_kv_scale",
    "no_sinks",
    "paged_attention",
    "paged_attention_fp8",
    "plan_status",
    "set_slot_check",
    "split_plan",
    "workspace_bytes",
    "workspace_bytes_max",
    "write_kv",
]
