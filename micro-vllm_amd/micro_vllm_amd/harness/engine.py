"""A minimal token-budgeted generation loop around the decoder model.

Scheduling follows the reference Scheduler's semantics (core/scheduler.py):
* each step has a token budget (`max_num_batched_tokens`) and a sequence cap
  (`max_num_seqs`);
* running requests are scheduled first, in order, each for
  min(pending tokens, remaining budget) tokens (:84-122), so long prompts are
  prefilled in chunks;
* when the block pool runs dry the newest running request is preempted: its
  blocks are freed, it goes back to the waiting queue, and it later
  recomputes its tokens (:100-113);
* waiting requests are then admitted first-in first-out while budget and
  sequence slots remain (:124-157);
* a request samples when its scheduled tokens reach the end of its known
  tokens; greedy decoding takes the first maximal logit (sampling/
  sampler.py:45-46) and a request finishes after `max_tokens` outputs
  (stop tokens are ignored).

Blocks come from a pool whose last id is the null block that pads block
tables (core/block.py:39; model_runner.py:243-245). With
`enable_prefix_cache=True` (config.py:112) complete blocks are indexed by
their chained digest after every step and a newly admitted request starts
after the longest indexed run of its blocks, sharing those physical blocks
with every other request that holds them (`block_pool.BlockPool`,
kv_cache_manager.py:113-222, scheduler.py:124-157). The step's flattened
input and attention metadata are built on the GPU
(`worker.packing.pack_scheduler_output`); sampling runs on the device with
one device-to-host copy of the sampled token ids per step.

Decode-only steps can run as HIP graphs, one per batch-size bucket, like the
reference's CUDA-graph execution (model_runner.py:344-497): the packing
kernels rewrite the bucket's static input buffers (padded the way
model_runner.py:78-122 pads them: no tokens past the real ones, slot -1,
null block ids) and the captured forward, greedy argmax included, is
replayed.

With `pipeline=True` the host runs one graph step ahead of the GPU: it
schedules and launches step k + 1 before reading step k's tokens back, so the
scheduling, packing and bookkeeping of one step overlap the previous step on
the GPU. Scheduling needs only token counts (a request finishes after
`max_tokens` outputs), so a token that is still on the GPU is carried as a
placeholder, -(1 + r) for row r of the previous step's samples, which the
captured graph replaces on the device with that step's sampled token. Before
any step that does not run as a graph, the pending step is read back and the
placeholders are filled in.
"""

from __future__ import annotations

import gc
import sys
import time
import weakref
from collections import deque
from dataclasses import dataclass, field

import numpy as np
import torch

from micro_vllm_amd.attention.spec import FullAttentionSpec
from micro_vllm_amd.harness.block_pool import BlockPool
from micro_vllm_amd.harness.model import DecoderModel
from micro_vllm_amd.harness.prefix_hash import BlockHashChain
from micro_vllm_amd.layers import argmax_rows
from micro_vllm_amd.worker.packing import (
    DeviceBlockRows,
    allocate_packed_batch,
    pack_decode_rows,
    pack_scheduler_output,
)
from micro_vllm_amd.worker.scheduler_output import (
    CacheGroupBlockTable,
    ScheduledRequest,
    SchedulerOutput,
)


@dataclass
class Request:
    request_id: str
    prompt_token_ids: list[int]
    max_tokens: int
    output_token_ids: list[int] = field(default_factory=list)
    num_computed_tokens: int = 0
    block_ids: list[int] = field(default_factory=list)

    def __post_init__(self) -> None:
        # Prompt followed by the outputs, grown in place (no per-step copies).
        self.token_ids: list[int] = list(self.prompt_token_ids) + list(self.output_token_ids)
        self._block_tuple: tuple[int, ...] | None = None
        # Prefix cache: digests of the complete blocks, and how many of the
        # request's leading blocks are indexed (or were a cache hit).
        self.hash_chain: BlockHashChain | None = None
        self.cached_blocks = 0
        # Device-resident block table: how many of block_ids the request's
        # row holds, and the first entry replaced since (None: none).
        self.row_sent = 0
        self.row_dirty: int | None = None

    def num_resolved_tokens(self) -> int:
        """Leading tokens that are real ids (pipelined mode appends
        placeholders for tokens still on the GPU, always at the end)."""

        n = len(self.token_ids)
        while n and self.token_ids[n - 1] < 0:
            n -= 1
        return n

    def append_output(self, token: int) -> None:
        self.output_token_ids.append(token)
        self.token_ids.append(token)

    def block_tuple(self) -> tuple[int, ...]:
        if self._block_tuple is None or len(self._block_tuple) != len(self.block_ids):
            self._block_tuple = tuple(self.block_ids)
        return self._block_tuple

    @property
    def num_known_tokens(self) -> int:
        return len(self.token_ids)

    @property
    def finished(self) -> bool:
        return len(self.output_token_ids) >= self.max_tokens


@dataclass
class GenerationResult:
    outputs: dict[str, list[int]]
    steps: int
    step_seconds: float
    output_tokens: int
    prompt_tokens: int
    preemptions: int
    decode_steps: int = 0          # steps whose requests all decode one token
    decode_seconds: float = 0.0
    prefix_hit_tokens: int = 0     # prompt tokens served by the prefix cache
    pack_seconds: float = 0.0      # host time spent packing steps (payload + launches)
    # Decode steps taken by the fast path (synchronous mode): how many, and
    # their host phases summed: schedule + pack + graph launch before the
    # GPU runs, bookkeeping while it runs, the wait for its tokens, and the
    # token appends after.
    fast_decode_steps: int = 0
    fast_phase_seconds: dict = field(default_factory=dict)

    @property
    def output_tokens_per_second(self) -> float:
        return self.output_tokens / self.step_seconds if self.step_seconds > 0 else 0.0


class GenerationEngine:
    """Continuous batching over one decoder model and its paged KV caches."""

    def __init__(
        self,
        model: DecoderModel,
        *,
        num_blocks: int,
        block_size: int = 16,
        max_num_batched_tokens: int = 8192,
        max_num_seqs: int = 256,
        max_model_len: int = 8192,
        decode_graphs: bool = False,
        pipeline: bool = False,
        enable_prefix_cache: bool = False,
        cache_namespace: str = "harness",
        incremental_block_table: bool = True,
    ) -> None:
        c = model.config
        self.model = model
        self.block_size = block_size
        self.max_model_len = max_model_len
        self.max_num_batched_tokens = max_num_batched_tokens
        self.max_num_seqs = max_num_seqs
        # Physical pool: ids [0, num_blocks - 1) are allocatable, the last id
        # is the null block used to pad block tables.
        self.num_blocks = num_blocks
        self.null_block_id = num_blocks - 1
        self.kv_caches = [
            torch.empty(
                (2, num_blocks, block_size, c.num_key_value_heads, c.head_dim),
                dtype=model.dtype,
                device=model.device,
            )
            for _ in range(c.num_hidden_layers)
        ]
        if getattr(model, "fused_layers", False):
            # Rotary rows for every position a request may reach.
            model.build_rotary_table(max_model_len)
        self.pool = BlockPool(num_blocks)
        self.enable_prefix_cache = enable_prefix_cache
        self.cache_namespace = cache_namespace
        self.prefix_hit_tokens = 0
        # Each running request's block ids live in a device row updated by
        # deltas (created on the first packed step).
        self.incremental_block_table = incremental_block_table
        self.block_rows: DeviceBlockRows | None = None
        self.pack_seconds = 0.0
        self._waiting: deque[Request] = deque()
        self._running: list[Request] = []
        self._requests: dict[str, Request] = {}
        self.preemptions = 0
        self.graphs = DecodeGraphs(self) if decode_graphs else None
        if pipeline and self.graphs is None:
            raise ValueError("pipeline=True needs decode_graphs=True")
        self.pipeline = pipeline
        # Synchronous decode-only steps skip the plan objects (see
        # _fast_decode_step); False forces every step through schedule().
        self.fast_decode = True
        # Arrays of the running requests carried from one fast step to the
        # next (valid while no other step changes the running set).
        self._fast_state: _FastState | None = None
        # Reused host (pinned) and device payload buffers of fast steps.
        self._fast_payload: tuple[torch.Tensor, torch.Tensor] | None = None
        self._fast_event: torch.cuda.Event | None = None
        self.fast_decode_steps = 0
        self.fast_phase_seconds = {"schedule": 0.0, "pack": 0.0, "replay": 0.0, "overlap": 0.0, "wait": 0.0,
                                   "append": 0.0}

    # ------------------------------------------------------------ requests
    def add_request(self, request: Request) -> None:
        if request.request_id in self._requests:
            raise ValueError(f"duplicate request id {request.request_id!r}")
        if not request.prompt_token_ids:
            raise ValueError("a request needs at least one prompt token")
        if len(request.prompt_token_ids) + request.max_tokens > self.max_model_len:
            raise ValueError(f"request {request.request_id!r} exceeds max_model_len {self.max_model_len}")
        self._requests[request.request_id] = request
        self._waiting.append(request)

    def has_unfinished_requests(self) -> bool:
        return bool(self._waiting or self._running)

    # ------------------------------------------------------------- blocks
    def _ensure_blocks(self, request: Request, num_tokens: int) -> bool:
        needed = -(-num_tokens // self.block_size) - len(request.block_ids)
        if needed <= 0:
            return True
        new = self.pool.allocate(needed)
        if new is None:
            return False
        request.block_ids.extend(new)
        return True

    def _free(self, request: Request) -> None:
        self.pool.release_all(request.block_ids)
        request.block_ids = []
        request._block_tuple = None
        request.cached_blocks = 0
        if self.block_rows is not None:
            self.block_rows.release(request.request_id)
        request.row_sent = 0
        request.row_dirty = None

    def _chain(self, request: Request) -> BlockHashChain:
        if request.hash_chain is None:
            request.hash_chain = BlockHashChain(
                block_size=self.block_size, cache_namespace=self.cache_namespace, vectorized=True
            )
        return request.hash_chain

    def _cache_hit(self, request: Request) -> list[int]:
        """Indexed blocks of the longest prefix of the request's first
        (known tokens - 1) // block_size blocks (kv_cache_manager.py:113-134,
        cache_group_manager.py:235-253)."""

        bs = self.block_size
        limit = min((request.num_known_tokens - 1) // bs, request.num_resolved_tokens() // bs)
        hit = []
        for digest in self._chain(request).extend(request.token_ids, max(limit, 0)):
            block = self.pool.lookup(digest)
            if block is None:
                break
            hit.append(block)
        return hit

    def _commit(self, request: Request) -> None:
        """Index the request's complete computed blocks; a block whose digest
        is indexed under another block is replaced by that canonical block
        (cache_group_manager.py:98-132)."""

        if not self.enable_prefix_cache:
            return
        full = min(request.num_computed_tokens, request.num_resolved_tokens()) // self.block_size
        if full <= request.cached_blocks:
            return
        digests = self._chain(request).extend(request.token_ids, full)
        for i in range(request.cached_blocks, full):
            block, digest = request.block_ids[i], digests[i]
            canonical = self.pool.lookup(digest)
            if canonical is None:
                self.pool.index(block, digest)
            elif canonical != block:
                self.pool.acquire(canonical)
                request.block_ids[i] = canonical
                self.pool.release(block)
                request._block_tuple = None
                request.row_dirty = i if request.row_dirty is None else min(request.row_dirty, i)
        request.cached_blocks = full

    # ----------------------------------------------------------- schedule
    def _scheduled(self, request: Request, num_tokens: int) -> ScheduledRequest:
        start = request.num_computed_tokens
        return ScheduledRequest(
            request_id=request.request_id,
            input_token_ids=tuple(request.token_ids[start : start + num_tokens]),
            num_computed_tokens=start,
            num_scheduled_tokens=num_tokens,
            requires_sampling=start + num_tokens == request.num_known_tokens,
            block_tables=(CacheGroupBlockTable(request.block_tuple()),),
        )

    def schedule(self) -> SchedulerOutput:
        self._fast_state = None
        budget = self.max_num_batched_tokens
        scheduled: list[ScheduledRequest] = []
        preempted: list[str] = []
        exhausted = False
        index = 0
        # Victims are popped from the end, so every request before `index`
        # stays in place.
        while index < len(self._running):
            request = self._running[index]
            index += 1
            if budget == 0 or len(scheduled) == self.max_num_seqs:
                break
            n = min(request.num_known_tokens - request.num_computed_tokens, budget)
            while not self._ensure_blocks(request, request.num_computed_tokens + n):
                if self._running[-1] is request:
                    break
                victim = self._running.pop()
                self._free(victim)
                victim.num_computed_tokens = 0
                self._waiting.append(victim)
                preempted.append(victim.request_id)
                self.preemptions += 1
            else:
                scheduled.append(self._scheduled(request, n))
                budget -= n
                continue
            if not scheduled:
                raise RuntimeError(f"request {request.request_id} cannot fit in the KV cache")
            exhausted = True
            break
        while (
            self._waiting
            and not exhausted
            and budget > 0
            and len(self._running) < self.max_num_seqs
        ):
            request = self._waiting[0]
            hit = self._cache_hit(request) if self.enable_prefix_cache else []
            computed = len(hit) * self.block_size
            n = min(request.num_known_tokens - computed, budget, self.max_model_len - computed)
            new = self.pool.allocate(-(-(computed + n) // self.block_size) - len(hit), hit)
            if new is None:
                if not scheduled:
                    raise RuntimeError(f"request {request.request_id} cannot fit in the KV cache")
                break
            request.block_ids = hit + new
            request._block_tuple = None
            request.num_computed_tokens = computed
            request.cached_blocks = len(hit)
            self.prefix_hit_tokens += computed
            scheduled.append(self._scheduled(request, n))
            budget -= n
            self._waiting.popleft()
            self._running.append(request)
        return SchedulerOutput(tuple(scheduled), tuple(preempted))

    def _update(self, plan: SchedulerOutput, sampled: list[int]) -> None:
        samples = iter(sampled)
        for item in plan.scheduled_requests:
            request = self._requests[item.request_id]
            request.num_computed_tokens += item.num_scheduled_tokens
            if item.requires_sampling:
                request.append_output(next(samples))
            self._commit(request)
            if item.requires_sampling and request.finished:
                self._running.remove(request)
                self._free(request)

    # ---------------------------------------------------------------- step
    def pack(self, plan: SchedulerOutput, into=None):
        """Pack a step on the GPU. With the incremental block table only the
        block ids that changed since a request's row was last written travel."""

        start = time.perf_counter()
        kwargs = {}
        if self.incremental_block_table:
            if self.block_rows is None:
                self.block_rows = DeviceBlockRows(
                    self.max_num_seqs, -(-self.max_model_len // self.block_size), self.model.device
                )
            updates = []
            for item in plan.scheduled_requests:
                request = self._requests[item.request_id]
                first = request.row_sent if request.row_dirty is None else min(request.row_sent, request.row_dirty)
                n = len(request.block_ids)
                if first < n:
                    updates.append((request.request_id, first, request.block_ids[first:n]))
                request.row_sent, request.row_dirty = n, None
            kwargs = dict(block_rows=self.block_rows, row_updates=updates)
        packed = pack_scheduler_output(
            plan,
            specs=[FullAttentionSpec()],
            block_size=self.block_size,
            null_block_id=self.null_block_id,
            device=self.model.device,
            into=into,
            **kwargs,
        )
        self.pack_seconds += time.perf_counter() - start
        return packed

    @torch.inference_mode()
    def execute(self, plan: SchedulerOutput) -> list[int]:
        """One model step on the GPU; returns the greedy tokens of the
        sampling requests, in plan order."""

        if self.graphs is not None and self.graphs.accepts(plan):
            return self.graphs.run(plan)
        packed = self.pack(plan)
        hidden = self.model.forward(packed.input_ids, packed.positions, self.kv_caches, packed.group_metadata[0])
        rows = packed.sampling_row_indices
        if rows.numel() == 0:
            return []
        logits = self.model.logits(hidden.index_select(0, rows))
        return argmax_rows(logits).tolist()

    def generate(self, requests: list[Request], progress_seconds: float | None = None) -> GenerationResult:
        """Run every request to completion. Synchronous mode times the
        synchronized steps (schedule + execute + update, as the reference
        benchmark times Engine.step, benchmarks/benchmark_engine.py:312-315);
        pipelined mode overlaps steps, so it times the whole loop, and a
        step's time is the wall time from its start to the next step's."""

        for request in requests:
            self.add_request(request)
        steps = decode_steps = 0
        seconds = decode_seconds = 0.0
        device = self.model.device
        torch.cuda.synchronize(device)
        pending: PendingStep | None = None
        loop_start = time.perf_counter()
        next_report = loop_start + progress_seconds if progress_seconds else None
        while self.has_unfinished_requests():
            if next_report is not None and time.perf_counter() >= next_report:
                done = sum(len(r.output_token_ids) for r in requests)
                print(f"[generate] step {steps}, {done} output tokens, {len(self._running)} running", file=sys.stderr, flush=True)
                next_report += progress_seconds
            start = time.perf_counter()
            if pending is None and not self.pipeline and self._fast_decode_step():
                elapsed = time.perf_counter() - start
                seconds += elapsed
                steps += 1
                decode_steps += 1
                decode_seconds += elapsed
                continue
            plan = self.schedule()
            if self.pipeline and self.graphs.accepts(plan):
                launched = self.graphs.launch(plan)
                if pending is not None:
                    self._resolve(pending)
                self._update_pending(plan, launched)
                pending = launched
            else:
                if pending is not None:
                    self._resolve(pending)
                    pending = None
                    plan = self._refresh(plan)
                sampled = self.execute(plan)
                torch.cuda.synchronize(device)
                self._update(plan, sampled)
            elapsed = time.perf_counter() - start
            seconds += elapsed
            steps += 1
            if all(s.num_scheduled_tokens == 1 for s in plan.scheduled_requests):
                decode_steps += 1
                decode_seconds += elapsed
        if pending is not None:
            self._resolve(pending)
        if self.pipeline:
            torch.cuda.synchronize(device)
            seconds = time.perf_counter() - loop_start
        return GenerationResult(
            outputs={r.request_id: list(r.output_token_ids) for r in requests},
            steps=steps,
            step_seconds=seconds,
            output_tokens=sum(len(r.output_token_ids) for r in requests),
            prompt_tokens=sum(len(r.prompt_token_ids) for r in requests),
            preemptions=self.preemptions,
            decode_steps=decode_steps,
            decode_seconds=decode_seconds,
            prefix_hit_tokens=self.prefix_hit_tokens,
            pack_seconds=self.pack_seconds,
            fast_decode_steps=self.fast_decode_steps,
            fast_phase_seconds=dict(self.fast_phase_seconds),
        )

    # ------------------------------------------------- decode fast path
    def _fast_decode_step(self) -> bool:
        """Run one decode-only graph step without building a plan, if the
        scheduler's plan would be exactly that; return False (nothing
        changed) otherwise.

        The plan is "every running request, one token, sampled" when no
        waiting request can be admitted (none waits, or every sequence slot
        is taken), every running request is decode-ready (one known token
        past its computed ones) and the pool holds every block the step needs
        (no preemption). The step then does what schedule() + execute() +
        _update() do, in the same order (blocks allocated in running order;
        per request: count, prefix-cache commit, finish and free), with the
        packing arrays held by numpy instead of one plan object per request:
        built from the requests, or carried from the previous fast step (each
        request one token further, finished ones dropped; any planned step
        discards them). The bookkeeping that does not need the sampled
        tokens runs while the GPU computes them; the tokens are appended
        after the step's device-to-host copy completes, so the step still
        ends synchronized with its tokens on the host."""

        g = self.graphs
        running = self._running
        n = len(running)
        if (
            not self.fast_decode
            or g is None
            or not self.incremental_block_table
            or n == 0
            or n > g.max_batch
            or n > self.max_num_batched_tokens
            or n > self.max_num_seqs
            or (self._waiting and n < self.max_num_seqs)
        ):
            return False
        t0 = time.perf_counter()
        bs = self.block_size
        state = self._fast_state
        if state is not None and state.running is running:
            # The previous fast step left every request one known token past
            # its computed ones; its arrays are this step's.
            computed, nblk, slots, tokens = state.computed, state.nblk, state.slots, state.tokens
            stale = set(state.dirty)
        else:
            computed = np.fromiter((r.num_computed_tokens for r in running), np.int64, n)
            known = np.fromiter((len(r.token_ids) for r in running), np.int64, n)
            if not np.array_equal(known - computed, np.ones(n, np.int64)):
                return False
            nblk = np.fromiter((len(r.block_ids) for r in running), np.int64, n)
            if self.block_rows is None:
                self.block_rows = DeviceBlockRows(self.max_num_seqs, -(-self.max_model_len // bs), self.model.device)
            slots = np.fromiter((self.block_rows.slot(r.request_id) for r in running), np.int64, n)
            tokens = np.fromiter((r.token_ids[-1] for r in running), np.int64, n)
            first = np.fromiter(
                (r.row_sent if r.row_dirty is None else min(r.row_sent, r.row_dirty) for r in running), np.int64, n
            )
            stale = set(np.nonzero(first < nblk)[0].tolist())
        self._fast_state = None
        short = np.nonzero(computed + 1 > nblk * bs)[0]
        if len(short):
            need = int(((computed[short] + bs) // bs - nblk[short]).sum())
            if need > self.pool.num_free_blocks:
                return False  # schedule() preempts
            nblk = nblk.copy()
            for i in short.tolist():
                if not self._ensure_blocks(running[i], int(computed[i]) + 1):
                    raise RuntimeError("block pool changed during a decode step")
                nblk[i] = len(running[i].block_ids)
                stale.add(i)
        rows = self.block_rows
        updates = []
        for i in sorted(stale):
            r = running[i]
            f = r.row_sent if r.row_dirty is None else min(r.row_sent, r.row_dirty)
            k = len(r.block_ids)
            if f < k:
                updates.append((int(slots[i]), f, r.block_ids[f:k]))
            r.row_sent, r.row_dirty = k, None

        size = g.bucket(n)
        entry = g.entries.get(size) or g.capture(size)
        t_pack = time.perf_counter()
        if self._fast_payload is None:
            words = 4096 + self.max_num_seqs * (2 + 8) + 4 * self.max_num_seqs
            self._fast_payload = (
                torch.empty(words, dtype=torch.int32, pin_memory=True),
                torch.empty(words, dtype=torch.int32, device=self.model.device),
            )
        with torch.inference_mode():
            pack_decode_rows(
                tokens, computed, nblk, slots, updates, spec=FullAttentionSpec(), block_size=bs,
                null_block_id=self.null_block_id, block_rows=rows, into=entry.buffers, staging=self._fast_payload,
            )
            t_replay = time.perf_counter()
            self.pack_seconds += t_replay - t_pack
            entry.graph.replay()
            host = g._host[g._flip]
            g._flip ^= 1
            host[:n].copy_(entry.tokens[:n], non_blocking=True)
            if self._fast_event is None:
                self._fast_event = torch.cuda.Event()
            done = self._fast_event
            done.record()
        t1 = time.perf_counter()

        # While the GPU runs: _update's per-request work that needs no token.
        finished = []
        dirty = []
        for i, r in enumerate(running):
            r.num_computed_tokens += 1
            if self.enable_prefix_cache:
                self._commit(r)
                if r.row_dirty is not None:
                    dirty.append(i)
            if len(r.output_token_ids) + 1 >= r.max_tokens:
                finished.append(i)
                self._free(r)
        # The next fast step's arrays, every request one token further (its
        # last tokens are filled in once this step's arrive).
        if finished:
            gone = set(finished)
            self._running = [r for i, r in enumerate(running) if i not in gone]
            keep = np.setdiff1d(np.arange(n), np.asarray(finished))
            remap = {int(old_i): new_i for new_i, old_i in enumerate(keep)}
            state = _FastState(
                self._running, computed[keep] + 1, nblk[keep], slots[keep], None,
                [remap[i] for i in dirty if i in remap],
            )
        else:
            keep = None
            state = _FastState(self._running, computed + 1, nblk, slots, None, dirty)
        t2 = time.perf_counter()
        done.synchronize()
        t3 = time.perf_counter()
        sampled = host[:n].numpy().copy()
        for r, token in zip(running, sampled.tolist()):
            r.output_token_ids.append(token)
            r.token_ids.append(token)
        state.tokens = sampled if keep is None else sampled[keep]
        self._fast_state = state
        t4 = time.perf_counter()
        ph = self.fast_phase_seconds
        ph["schedule"] += t_pack - t0
        ph["pack"] += t_replay - t_pack
        ph["replay"] += t1 - t_replay
        ph["overlap"] += t2 - t1
        ph["wait"] += t3 - t2
        ph["append"] += t4 - t3
        self.fast_decode_steps += 1
        return True

    # ------------------------------------------------------- pipelining
    def _update_pending(self, plan: SchedulerOutput, step: "PendingStep") -> None:
        """_update for a launched graph step whose tokens are still on the
        GPU: every request gets a placeholder for its token."""

        for row, item in enumerate(plan.scheduled_requests):
            request = self._requests[item.request_id]
            request.num_computed_tokens += 1
            request.append_output(-(1 + row))
            step.slots.append((request, len(request.output_token_ids) - 1))
            self._commit(request)
            if request.finished:
                self._running.remove(request)
                self._free(request)

    def _resolve(self, step: "PendingStep") -> None:
        """Replace a launched step's placeholders with its sampled tokens."""

        step.event.synchronize()
        values = step.host[: len(step.slots)].tolist()
        for (request, index), token in zip(step.slots, values):
            request.output_token_ids[index] = token
            request.token_ids[len(request.prompt_token_ids) + index] = token

    def _refresh(self, plan: SchedulerOutput) -> SchedulerOutput:
        """The plan's input ids re-read after placeholders were resolved."""

        items = []
        for item in plan.scheduled_requests:
            request = self._requests[item.request_id]
            start = item.num_computed_tokens
            items.append(
                ScheduledRequest(
                    request_id=item.request_id,
                    input_token_ids=tuple(request.token_ids[start : start + item.num_scheduled_tokens]),
                    num_computed_tokens=start,
                    num_scheduled_tokens=item.num_scheduled_tokens,
                    requires_sampling=item.requires_sampling,
                    block_tables=item.block_tables,
                )
            )
        return SchedulerOutput(tuple(items), plan.preempted_request_ids)


class DecodeGraphs:
    """Captured decode steps of one engine, one HIP graph per bucket."""

    BUCKETS = (1, 2, 4, 8, 16, 32, 64, 128, 256, 512)

    def __init__(self, engine: GenerationEngine) -> None:
        # A weak reference: the engine owns this object, and a cycle between
        # them would leave the captured graphs to the cyclic collector, which
        # may run inside a later capture, where destroying a graph and
        # freeing its memory pool is not allowed (the process aborts).
        self._engine = weakref.ref(engine)
        self.width = -(-engine.max_model_len // engine.block_size)
        self.max_batch = self.BUCKETS[-1]
        self.pool = torch.cuda.graph_pool_handle()
        self.entries: dict[int, DecodeGraph] = {}
        device = engine.model.device
        # The sampled tokens of the latest graph step, read by the next one
        # through placeholders (pipelined mode).
        self.last_tokens = torch.zeros(self.max_batch, dtype=torch.int64, device=device)
        self._host = [torch.empty(self.max_batch, dtype=torch.int64, pin_memory=True) for _ in range(2)]
        self._flip = 0

    @property
    def engine(self) -> GenerationEngine:
        engine = self._engine()
        if engine is None:
            raise RuntimeError("the engine of these decode graphs no longer exists")
        return engine

    def accepts(self, plan: SchedulerOutput) -> bool:
        items = plan.scheduled_requests
        return (
            0 < len(items) <= self.max_batch
            and all(s.num_scheduled_tokens == 1 and s.requires_sampling for s in items)
        )

    def bucket(self, num_requests: int) -> int:
        return min(b for b in self.BUCKETS if b >= num_requests)

    def _pack(self, plan: SchedulerOutput, buffers) -> None:
        self.engine.pack(plan, into=buffers)

    def forward(self, buffers) -> tuple[torch.Tensor, torch.Tensor]:
        """The decode step on a bucket's buffers: logits and greedy token of every row."""

        model = self.engine.model
        # Placeholder ids -(1 + r) stand for the token sampled at row r of
        # the previous step (resolved inside the embedding lookup).
        hidden = model.forward(
            buffers.input_ids, buffers.positions, self.engine.kv_caches, buffers.group_metadata[0],
            placeholder_tokens=self.last_tokens,
        )
        logits = model.logits(hidden)
        tokens = argmax_rows(logits, copy_into=self.last_tokens)
        return logits, tokens

    @torch.inference_mode()
    def capture(self, size: int) -> "DecodeGraph":
        e = self.engine
        buffers = allocate_packed_batch(
            num_groups=1,
            block_size=e.block_size,
            token_capacity=size,
            request_capacity=size,
            block_table_widths=[self.width],
            sampling_capacity=size,
            device=e.model.device,
            max_query_len=1,
        )
        self._pack(SchedulerOutput(()), buffers)  # an all-padding step: writes nothing
        # The warm-up forwards overwrite the previous step's sampled tokens,
        # which a pipelined step launched right after the capture still reads.
        saved_tokens = self.last_tokens.clone()
        side = torch.cuda.Stream(e.model.device)
        side.wait_stream(torch.cuda.current_stream(e.model.device))
        with torch.cuda.stream(side):
            for _ in range(2):
                self.forward(buffers)
        torch.cuda.current_stream(e.model.device).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        # Whatever dead objects still hold graphs or device memory are freed
        # here, and the cyclic collector stays off during the capture: a
        # graph destroyed inside another capture aborts the process.
        gc.collect()
        collecting = gc.isenabled()
        gc.disable()
        try:
            with torch.cuda.graph(graph, pool=self.pool):
                logits, tokens = self.forward(buffers)
        finally:
            if collecting:
                gc.enable()
        self.last_tokens.copy_(saved_tokens)
        entry = DecodeGraph(graph, buffers, logits, tokens)
        self.entries[size] = entry
        return entry

    @torch.inference_mode()
    def run(self, plan: SchedulerOutput) -> list[int]:
        n = len(plan.scheduled_requests)
        size = self.bucket(n)
        entry = self.entries.get(size) or self.capture(size)
        self._pack(plan, entry.buffers)
        entry.graph.replay()
        return entry.tokens[:n].tolist()

    @torch.inference_mode()
    def launch(self, plan: SchedulerOutput) -> "PendingStep":
        """Replay the plan's graph and start copying its tokens to the host
        without waiting for them (pipelined mode)."""

        n = len(plan.scheduled_requests)
        size = self.bucket(n)
        entry = self.entries.get(size) or self.capture(size)
        self._pack(plan, entry.buffers)
        entry.graph.replay()
        host = self._host[self._flip]  # alternates: the previous step's buffer is read after this launch
        self._flip ^= 1
        host[:n].copy_(entry.tokens[:n], non_blocking=True)
        event = torch.cuda.Event()
        event.record()
        return PendingStep(host, event)


@dataclass
class _FastState:
    """Arrays of the running requests, in order, carried between fast decode
    steps: computed tokens, block counts, block-row slots, last tokens, and
    the indices whose block rows the prefix cache changed."""

    running: list
    computed: np.ndarray
    nblk: np.ndarray
    slots: np.ndarray
    tokens: np.ndarray
    dirty: list


@dataclass
class PendingStep:
    """A launched graph step: its tokens arrive in `host` once `event`
    completes; `slots` lists the (request, output index) placeholders."""

    host: torch.Tensor
    event: torch.cuda.Event
    slots: list = field(default_factory=list)


@dataclass
class DecodeGraph:
    graph: torch.cuda.CUDAGraph
    buffers: object   # the bucket's PackedBatch (static inputs)
    logits: torch.Tensor
    tokens: torch.Tensor
