"""GPU packing parity (bit-exact) against the reference's literal vectors and
the oracle packing, including per-group metadata, graph padding and
randomised plans; plus GPU context starts."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _golden import GOLDEN, SPEC_KINDS, requests_from_case
from micro_vllm_amd.attention import Attention, ChunkedLocalSpec, FullAttentionSpec, SlidingWindowSpec
from micro_vllm_amd.attention.attention import context_starts
from micro_vllm_amd.worker.packing import pack_scheduler_output
from micro_vllm_amd.worker.scheduler_output import CacheGroupBlockTable, ScheduledRequest, SchedulerOutput

pytestmark = pytest.mark.gpu

SPEC_OBJECTS = {
    "full": lambda p: FullAttentionSpec(),
    "sliding_window": lambda p: SlidingWindowSpec(p),
    "chunked_local": lambda p: ChunkedLocalSpec(p),
}


def plan_from(requests: list[oracle.Request]) -> SchedulerOutput:
    return SchedulerOutput(
        tuple(
            ScheduledRequest(
                request_id=r.request_id,
                input_token_ids=r.input_token_ids,
                num_computed_tokens=r.num_computed_tokens,
                num_scheduled_tokens=r.num_scheduled_tokens,
                requires_sampling=r.requires_sampling,
                block_tables=tuple(CacheGroupBlockTable(g) for g in r.block_tables),
            )
            for r in requests
        )
    )


def check_against_oracle(packed, requests, specs, *, block_size, null_block_id, capacities=None):
    for g, spec in enumerate(specs):
        expected = oracle.pack(requests, group=g, block_size=block_size, null_block_id=null_block_id, spec=spec.kernel_code())
        if capacities:
            expected = oracle.graph_pad(expected, null_block_id=null_block_id, **capacities)
        md = packed.group_metadata[g]
        got = {
            "positions": md.query_positions,
            "context_starts": md.query_context_start_positions,
            "query_start_locations": md.query_start_locations,
            "context_lengths": md.context_lengths,
            "block_table": md.block_table,
            "slot_mapping": md.slot_mapping,
        }
        if g == 0:
            got["input_ids"] = packed.input_ids
            got["sampling_row_indices"] = packed.sampling_row_indices
        for name, tensor in got.items():
            assert tensor.dtype == torch.int64, name
            assert tensor.cpu().numpy().tolist() == expected[name].tolist(), (g, name)


@pytest.mark.parametrize("c", GOLDEN["packing_cases"], ids=lambda c: c["name"])
def test_packing_golden_vectors(device, c):
    requests = requests_from_case(c)
    specs = [SPEC_OBJECTS[g["spec"][0]](g["spec"][1]) for g in c.get("groups", [{"spec": ["full", 0]}])]
    caps = None
    kwargs = {}
    if "graph" in c:
        width = max(len(r.block_tables[0]) for r in requests)
        caps = dict(token_capacity=c["graph"]["token_capacity"], request_capacity=c["graph"]["request_capacity"], block_table_width=width)
        kwargs = caps
    packed = pack_scheduler_output(
        plan_from(requests), specs=specs, block_size=c["block_size"], null_block_id=c["null_block_id"], device=device, **kwargs
    )
    torch.cuda.synchronize()
    check_against_oracle(packed, requests, specs, block_size=c["block_size"], null_block_id=c["null_block_id"], capacities=caps)
    expect = c.get("expect", {})
    md = packed.group_metadata[0]
    if "slot_mapping" in expect:
        assert md.slot_mapping.tolist() == expect["slot_mapping"]
    if "block_table" in expect:
        assert md.block_table.tolist() == expect["block_table"]
    if "query_start_locations" in expect:
        assert md.query_start_locations.tolist() == expect["query_start_locations"]
    if "input_ids" in expect:
        assert packed.input_ids.tolist() == expect["input_ids"]
    if "last_slot" in expect:
        assert md.slot_mapping[-1].item() == expect["last_slot"]
    if "block_table_shape" in expect:
        assert list(md.block_table.shape) == expect["block_table_shape"]
    for g, eg in enumerate(c.get("expect_groups", [])):
        m = packed.group_metadata[g]
        if "context_starts" in eg:
            assert m.query_context_start_positions.tolist() == eg["context_starts"]
        assert m.block_table.tolist() == eg["block_table"]
        assert m.slot_mapping.tolist() == eg["slot_mapping"]
    if len(packed.group_metadata) > 1:
        assert packed.group_metadata[1].query_positions is packed.group_metadata[0].query_positions
        assert packed.group_metadata[1].query_start_locations is packed.group_metadata[0].query_start_locations


def random_requests(rng, num_requests, num_groups, block_size):
    requests = []
    for i in range(num_requests):
        computed = int(rng.integers(0, 3000))
        scheduled = int(rng.choice([1, 1, 1, int(rng.integers(1, 600))]))
        total = computed + scheduled
        tables = []
        for _ in range(num_groups):
            n = -(-total // block_size) + int(rng.integers(0, 3))  # some requests hold extra blocks
            tables.append(tuple(int(x) for x in rng.integers(0, 100_000, n)))
        requests.append(
            oracle.Request(
                request_id=f"r{i}",
                input_token_ids=tuple(int(x) for x in rng.integers(0, 151_936, scheduled)),
                num_computed_tokens=computed,
                num_scheduled_tokens=scheduled,
                requires_sampling=bool(rng.integers(0, 2)),
                block_tables=tuple(tables),
            )
        )
    return requests


@pytest.mark.parametrize("num_requests", [0, 1, 7, 256, 1500])
@pytest.mark.parametrize("padded", [False, True])
def test_random_plans_match_oracle(device, num_requests, padded):
    rng = np.random.default_rng(num_requests + 7 * padded)
    block_size = 16
    specs = [FullAttentionSpec(), SlidingWindowSpec(int(rng.integers(1, 500))), ChunkedLocalSpec(int(rng.integers(1, 500)))]
    requests = random_requests(rng, num_requests, len(specs), block_size)
    kwargs, caps = {}, None
    if padded:
        tokens = sum(r.num_scheduled_tokens for r in requests)
        width = max((len(t) for r in requests for t in r.block_tables), default=0) + 5
        caps = dict(token_capacity=tokens + 37, request_capacity=num_requests + 3, block_table_width=width)
        kwargs = caps
    packed = pack_scheduler_output(plan_from(requests), specs=specs, block_size=block_size, null_block_id=100_000, device=device, **kwargs)
    torch.cuda.synchronize()
    if not padded:
        check_against_oracle(packed, requests, specs, block_size=block_size, null_block_id=100_000)
        return
    for g, spec in enumerate(specs):
        expected = oracle.pack(requests, group=g, block_size=block_size, null_block_id=100_000, spec=spec.kernel_code())
        expected = oracle.graph_pad(expected, null_block_id=100_000, **caps)
        md = packed.group_metadata[g]
        assert md.block_table.cpu().numpy().tolist() == expected["block_table"].tolist()
        assert md.slot_mapping.cpu().numpy().tolist() == expected["slot_mapping"].tolist()
        assert md.query_context_start_positions.cpu().numpy().tolist() == expected["context_starts"].tolist()
        assert md.query_start_locations.cpu().numpy().tolist() == expected["query_start_locations"].tolist()
        assert md.context_lengths.cpu().numpy().tolist() == expected["context_lengths"].tolist()
        assert md.query_positions.cpu().numpy().tolist() == expected["positions"].tolist()
    assert packed.input_ids.cpu().numpy().tolist() == expected["input_ids"].tolist()


@pytest.mark.parametrize("c", GOLDEN["spec_cases"], ids=lambda c: f"{c['spec'][0]}-{c['spec'][1]}-{c['positions']}")
def test_context_starts_golden_vectors(device, c):
    spec = SPEC_OBJECTS[c["spec"][0]](c["spec"][1])
    got = context_starts(torch.tensor(c["positions"], device=device), spec)
    assert got.tolist() == c["expect"]


def test_build_metadata_keeps_inputs_and_computes_starts(device):
    positions = torch.tensor([2, 3, 4, 5], device=device)
    args = dict(
        query_positions=positions,
        query_start_locations=torch.tensor([0, 4], device=device),
        context_lengths=torch.tensor([6], device=device),
        block_table=torch.tensor([[0, 1]], device=device),
        slot_mapping=torch.tensor([2, 3, 4, 5], device=device),
        block_size=4,
    )
    md = Attention(SlidingWindowSpec(3), "mi355x_paged").build_metadata(**args)
    assert md.query_positions is positions
    assert md.block_table is args["block_table"]
    assert md.query_context_start_positions.tolist() == [0, 1, 2, 3]
    big = torch.arange(0, 1_000_000, 7, device=device)
    got = context_starts(big, ChunkedLocalSpec(13)).cpu().numpy()
    assert np.array_equal(got, oracle.context_starts(oracle.CHUNKED_LOCAL, 13, big.cpu().numpy()))


# ------------------------------------------ device-resident block rows (deltas)


def test_device_block_rows_give_the_oracle_packing_over_steps(device):
    """A device-resident block table updated by deltas (appended ids,
    a replaced entry, a released row reused by another request) packs every
    step bit-identically to the oracle packing of the full lists, unpadded
    and at graph capacities."""

    from micro_vllm_amd.worker.packing import DeviceBlockRows, allocate_packed_batch

    rng = np.random.default_rng(12)
    rows = DeviceBlockRows(num_slots=4, width=48, device=device)
    null = 999
    lists = {"a": rng.permutation(500)[:20].tolist(), "b": rng.permutation(500)[:3].tolist()}
    sent = {"a": 0, "b": 0}
    computed = {"a": 300, "b": 40}
    steps = [
        dict(),                                   # both rows written from scratch
        dict(append={"a": 1}),                    # one appended id
        dict(replace={"a": 5}),                   # a replaced entry (prefix-cache dedup)
        dict(release="b", admit=("c", 7)),        # b leaves, c takes its row
        dict(append={"c": 2, "a": 1}),
    ]
    buffers = allocate_packed_batch(num_groups=1, block_size=16, token_capacity=8, request_capacity=4,
                                    block_table_widths=[48], sampling_capacity=4, device=device, max_query_len=4)
    for step in steps:
        updates = []
        for rid, n in step.get("append", {}).items():
            lists[rid].extend(rng.integers(500, 900, size=n).tolist())
        for rid, i in step.get("replace", {}).items():
            lists[rid][i] = 901
            sent[rid] = min(sent[rid], i)
        if "release" in step:
            rows.release(step["release"])
            del lists[step["release"]], computed[step["release"]]
            rid, n = step["admit"]
            lists[rid], sent[rid], computed[rid] = rng.permutation(500)[:n].tolist(), 0, 90
        for rid, ids in lists.items():
            if sent[rid] < len(ids):
                updates.append((rid, sent[rid], ids[sent[rid]:]))
                sent[rid] = len(ids)
        requests = []
        for rid, ids in lists.items():
            q = 1 if rid != "c" else 3
            pos0 = min(computed[rid], len(ids) * 16 - q)
            requests.append(oracle.Request(rid, tuple(range(q)), pos0, q, True, (tuple(ids),)))
        plan = plan_from(requests)
        for into, caps in ((None, None), (buffers, dict(token_capacity=8, request_capacity=4, block_table_width=48))):
            packed = pack_scheduler_output(plan, specs=[FullAttentionSpec()], block_size=16, null_block_id=null,
                                           device=device, into=into, block_rows=rows, row_updates=updates)
            torch.cuda.synchronize()
            check_against_oracle(packed, requests, [FullAttentionSpec()], block_size=16, null_block_id=null, capacities=caps)
            updates = []  # the rows already hold them for the padded pass


def test_decode_rows_packing_equals_the_plan_packing(device):
    """``pack_decode_rows`` (a decode-only step packed from per-request
    arrays, the engine's fast path) writes exactly what
    ``pack_scheduler_output`` writes for the same decode plan: every buffer
    of a graph bucket bit-identical, with row updates (new rows, appended
    ids, a replaced entry) applied to the device-resident table the same
    way, over several steps."""

    from micro_vllm_amd.worker.packing import DeviceBlockRows, allocate_packed_batch, pack_decode_rows

    rng = np.random.default_rng(31)
    null, width, cap = 4999, 40, 16
    rows_a = DeviceBlockRows(num_slots=cap, width=width, device=device)
    rows_b = DeviceBlockRows(num_slots=cap, width=width, device=device)
    bufs = [allocate_packed_batch(num_groups=1, block_size=16, token_capacity=cap, request_capacity=cap,
                                  block_table_widths=[width], sampling_capacity=cap, device=device, max_query_len=1)
            for _ in range(2)]
    reqs = {f"r{i}": dict(ids=rng.permutation(4000)[: int(rng.integers(1, 30))].tolist(), sent=0) for i in range(11)}
    for step in range(4):
        if step == 2:
            reqs["r3"]["ids"][1] = 4100      # prefix-cache switch to a canonical block
            reqs["r3"]["sent"] = 1
        if step == 3:
            reqs["r5"]["ids"].append(4200)  # a new block
        names = list(reqs)
        computed = np.array([len(reqs[k]["ids"]) * 16 - int(rng.integers(1, 16)) for k in names], np.int64)
        tokens = rng.integers(0, 50_000, size=len(names)).astype(np.int64)
        updates = [(k, reqs[k]["sent"], reqs[k]["ids"][reqs[k]["sent"]:]) for k in names
                   if reqs[k]["sent"] < len(reqs[k]["ids"])]
        for k in names:
            reqs[k]["sent"] = len(reqs[k]["ids"])
        items = [
            ScheduledRequest(k, (int(t),), int(c), 1, True, (CacheGroupBlockTable(tuple(reqs[k]["ids"])),))
            for k, t, c in zip(names, tokens, computed)
        ]
        a = pack_scheduler_output(SchedulerOutput(tuple(items)), specs=[FullAttentionSpec()], block_size=16,
                                  null_block_id=null, device=device, into=bufs[0], block_rows=rows_a,
                                  row_updates=updates)
        slots = np.array([rows_b.slot(k) for k in names], np.int64)
        b = pack_decode_rows(
            tokens, computed, np.array([len(reqs[k]["ids"]) for k in names], np.int64), slots,
            [(rows_b.slot(k), f, ids) for k, f, ids in updates], spec=FullAttentionSpec(), block_size=16,
            null_block_id=null, block_rows=rows_b, into=bufs[1],
        )
        torch.cuda.synchronize()
        assert torch.equal(rows_a.rows, rows_b.rows)
        for x, y in ((a.input_ids, b.input_ids), (a.positions, b.positions),
                     (a.sampling_row_indices, b.sampling_row_indices)):
            assert torch.equal(x, y)
        ma, mb = a.group_metadata[0], b.group_metadata[0]
        for f in ("query_context_start_positions", "query_start_locations", "context_lengths", "block_table",
                  "slot_mapping"):
            assert torch.equal(getattr(ma, f), getattr(mb, f)), (step, f)
        assert b.input_ids[: len(names)].tolist() == tokens.tolist()

