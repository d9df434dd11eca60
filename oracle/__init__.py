"""CPU oracle for the ragged paged-attention path (TEST INFRASTRUCTURE ONLY).

A numpy restatement of the reference's attention operator and packing code,
used only by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py``, as the reference results the HIP path is compared with.
The HIP library never imports it.

Every function is pinned against the reference tests' literal vectors and
against closed forms in ``tests/test_oracle.py``; none is left unpinned.
"""

from .numerics import (  # noqa: F401
    BF16,
    F16,
    F32,
    bf16_bits_to_f32,
    f32_to_bf16_bits,
    from_f32,
    to_f32,
)
from .paged_attention import (  # noqa: F401
    CHUNKED_LOCAL,
    FULL,
    SLIDING_WINDOW,
    Batch,
    context_start,
    context_starts,
    dense_attention,
    gather_kv_cache,
    make_batch,
    map_cache_slots,
    reference_forward,
    write_kv_cache,
)
from .packing import (  # noqa: F401
    Request,
    build_block_table,
    build_slot_mapping,
    flatten_model_input,
    graph_pad,
    pack,
)
