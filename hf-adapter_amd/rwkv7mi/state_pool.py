"""Serving state-slot pool: persistent, layer-major recurrent state indexed by
scheduler slots, with graph-bucketed decode over arbitrary slot sets.

Follows the serving ABI of docs/integrations/RWKV7_STATE_CACHE_ABI.md:52-133
(the reference describes it; NativeRWKV7Cache's select_batch / reorder /
reset, rwkv7_hf/model_cache.py:335-343, 368, are its dense-batch
semantics):

* storage ``state [L, C + 1, H, N, N]`` (fp32), ``xpa / xpf [L, C + 1, D]``,
  ``v_first [C + 1, A]``, ``seen_tokens [C + 1]``; slot ``C`` is a scratch
  slot that padded graph rows read and never write;
* ``allocate`` returns zeroed, uniquely owned slots with a generation;
  ``free`` checks the generation and bumps it, so a stale handle cannot
  touch a reassigned slot; ``reset`` / ``clone`` / ``gather`` / ``scatter`` /
  ``snapshot`` / ``restore`` as the ABI lists them;
* :class:`PooledDecoder` runs one decode step for any list of live slots:
  the rows are gathered into a graph bucket's layer-major batch cache (one
  ``rwkv7mi_slot_copy`` launch per tensor family for all layers), the
  bucket's captured hipGraph replays, and only the active rows are
  scattered back; padding rows use the scratch slot with active = 0.

Every copy is the HIP slot-copy kernel (byte moves, bit-exact).
"""
from __future__ import annotations

import ctypes
import hashlib

import torch

from . import _lib

LAYOUT_VERSION = "rwkv7mi.state_pool.v1"


def _ptr_i64(t):
    return None if t is None else _lib.ptr(t)


def _slot_copy(src, src_layer, src_row, src_rows, dst, dst_layer, dst_row, dst_rows, active, nrows, row_bytes,
               nlayers, stream):
    _lib.call("rwkv7mi_slot_copy", None if src is None else ctypes.c_void_p(src), int(src_layer), int(src_row),
              _ptr_i64(src_rows), ctypes.c_void_p(dst), int(dst_layer), int(dst_row), _ptr_i64(dst_rows),
              _ptr_i64(active), int(nrows), int(row_bytes), int(nlayers), stream)


def _layer_major(tensors) -> int | None:
    """Byte stride between consecutive layers' tensors when they are equally
    spaced contiguous views (None otherwise)."""
    if not all(t.is_contiguous() for t in tensors):
        return None
    if len(tensors) == 1:
        return 0
    d = tensors[1].data_ptr() - tensors[0].data_ptr()
    for a, b in zip(tensors, tensors[1:]):
        if b.data_ptr() - a.data_ptr() != d:
            return None
    return d


class RWKV7StatePool:
    """Layer-major state pool of ``capacity`` request slots (plus one scratch slot)."""

    def __init__(self, config, capacity: int, *, device="cuda", dtype=torch.float16):
        if capacity < 1:
            raise ValueError("capacity must be positive")
        self.config = config
        self.capacity = int(capacity)
        self.device = torch.device(device)
        self.dtype = dtype
        L, H, N, D, A = (config.num_hidden_layers, config.num_heads, config.head_dim, config.hidden_size,
                         config.attention_hidden_size)
        C = self.capacity + 1
        self.state = torch.zeros(L, C, H, N, N, device=self.device, dtype=torch.float32)
        self.xpa = torch.zeros(L, C, D, device=self.device, dtype=dtype)
        self.xpf = torch.zeros(L, C, D, device=self.device, dtype=dtype)
        self.v_first = torch.zeros(C, A, device=self.device, dtype=dtype)
        self.seen_tokens = [0] * C
        self.generation = [0] * C
        self.allocated = [False] * C
        self.owner: dict[int, object] = {}
        self.scratch_slot = self.capacity

    # ------------------------------------------------------------ bookkeeping
    @property
    def bytes_per_slot(self) -> int:
        c = self.config
        return (c.num_hidden_layers * c.num_heads * c.head_dim * c.head_dim * 4
                + 2 * c.num_hidden_layers * c.hidden_size * self.xpa.element_size()
                + c.attention_hidden_size * self.v_first.element_size())

    def free_slots(self) -> int:
        return sum(1 for s in range(self.capacity) if not self.allocated[s])

    def _idx(self, slots) -> torch.Tensor:
        return torch.as_tensor(list(slots), dtype=torch.int64).to(self.device, non_blocking=True)

    def check(self, slots, generations=None, *, live: bool = True) -> None:
        """Slots are distinct, in range and (``live``) allocated, with matching generations."""
        slots = [int(s) for s in slots]
        if len(set(slots)) != len(slots):
            raise ValueError(f"duplicate destination slots {slots}")
        for i, s in enumerate(slots):
            if not 0 <= s < self.capacity:
                raise ValueError(f"slot {s} out of range (capacity {self.capacity})")
            if live and not self.allocated[s]:
                raise ValueError(f"slot {s} is not allocated")
            if generations is not None and int(generations[i]) != self.generation[s]:
                raise ValueError(f"slot {s}: stale handle (generation {generations[i]}, slot is at "
                                 f"{self.generation[s]})")

    # ------------------------------------------------------------ allocator
    def allocate(self, request_ids) -> list[tuple[int, int]]:
        """Zeroed, uniquely owned slots: ``[(slot, generation), ...]``."""
        request_ids = list(request_ids)
        free = [s for s in range(self.capacity) if not self.allocated[s]]
        if len(free) < len(request_ids):
            raise RuntimeError(f"state pool full: {len(request_ids)} requested, {len(free)} free")
        slots = free[:len(request_ids)]
        for s, rid in zip(slots, request_ids):
            self.allocated[s] = True
            self.owner[s] = rid
        self.reset(slots)
        return [(s, self.generation[s]) for s in slots]

    def free(self, slots, generations) -> None:
        """Invalidate the handles, then make the slots reusable."""
        self.check(slots, generations)
        for s in slots:
            self.generation[int(s)] += 1
            self.allocated[int(s)] = False
            self.owner.pop(int(s), None)

    def _rows(self, slots, *, zero=False, src_slots=None):
        """One slot-copy launch per tensor family: pool rows ``src_slots`` (or
        zeros) into pool rows ``slots``."""
        n = len(slots)
        if n == 0:
            return
        dst = self._idx(slots)
        src = None if zero else self._idx(src_slots)
        st = _lib.stream_of(self.state)
        for t in (self.state, self.xpa, self.xpf):
            row = t[0, 0].numel() * t.element_size()
            layer = t[0].numel() * t.element_size()
            _slot_copy(None if zero else t.data_ptr(), layer, row, src, t.data_ptr(), layer, row, dst, None, n, row,
                       t.shape[0], st)
        vrow = self.v_first[0].numel() * self.v_first.element_size()
        _slot_copy(None if zero else self.v_first.data_ptr(), 0, vrow, src, self.v_first.data_ptr(), 0, vrow, dst,
                   None, n, vrow, 1, st)

    def reset(self, slots) -> None:
        """Exact new-request state (zeros, seen_tokens 0)."""
        self.check(slots)
        self._rows(list(slots), zero=True)
        for s in slots:
            self.seen_tokens[int(s)] = 0

    def clone(self, source_slots, destination_slots) -> None:
        """Deep copy (beam fork, prefix copy-on-write)."""
        self.check(source_slots)
        self.check(destination_slots)
        if set(map(int, source_slots)) & set(map(int, destination_slots)):
            raise ValueError("clone: source and destination slots overlap")
        self._rows(list(destination_slots), src_slots=list(source_slots))
        for s, d in zip(source_slots, destination_slots):
            self.seen_tokens[int(d)] = self.seen_tokens[int(s)]

    # ------------------------------------------------------------ per layer
    def gather(self, layer_id: int, slot_ids):
        """``(state [B,H,N,N], xpa [B,D], xpf [B,D])`` of one layer (new tensors)."""
        self.check(slot_ids)
        idx = self._idx(slot_ids)
        out = []
        st = _lib.stream_of(self.state)
        for t in (self.state, self.xpa, self.xpf):
            o = torch.empty((len(slot_ids),) + tuple(t.shape[2:]), device=self.device, dtype=t.dtype)
            row = t[0, 0].numel() * t.element_size()
            _slot_copy(t[layer_id].data_ptr(), 0, row, idx, o.data_ptr(), 0, row, None, None, len(slot_ids), row, 1, st)
            out.append(o)
        return tuple(out)

    def scatter(self, layer_id: int, slot_ids, updated, active=None) -> None:
        """Commit one layer's ``(state, xpa, xpf)`` rows to exactly those live slots."""
        self.check(slot_ids)
        idx = self._idx(slot_ids)
        act = None if active is None else torch.as_tensor(active, dtype=torch.uint8).to(self.device)
        st = _lib.stream_of(self.state)
        for t, u in zip((self.state, self.xpa, self.xpf), updated):
            u = u.contiguous()
            row = t[0, 0].numel() * t.element_size()
            _slot_copy(u.data_ptr(), 0, row, None, t[layer_id].data_ptr(), 0, row, idx, act, len(slot_ids), row, 1, st)

    # ------------------------------------------------------------ whole batches
    def _batch_copy(self, cache, rows, *, to_cache: bool, active=None) -> None:
        if cache._state and cache._state[0].dtype != self.state.dtype:
            raise ValueError(f"the state pool holds {self.state.dtype} states; got a cache with a "
                             f"{cache._state[0].dtype} state")
        n = len(rows)
        idx = self._idx(rows)
        act = None if active is None else torch.as_tensor(active, dtype=torch.uint8).to(self.device)
        st = _lib.stream_of(self.state)
        for pool_t, layers in ((self.state, cache._state), (self.xpa, cache._xpa), (self.xpf, cache._xpf)):
            row = pool_t[0, 0].numel() * pool_t.element_size()
            pl = pool_t[0].numel() * pool_t.element_size()
            cl = _layer_major(layers)
            groups = [(layers[0], pool_t.data_ptr(), cl, len(layers))] if cl is not None else \
                [(t, pool_t[i].data_ptr(), 0, 1) for i, t in enumerate(layers)]
            for t0, pbase, cstride, nl in groups:
                if to_cache:
                    _slot_copy(pbase, pl, row, idx, t0.data_ptr(), cstride, row, None, None, n, row, nl, st)
                else:
                    _slot_copy(t0.data_ptr(), cstride, row, None, pbase, pl, row, idx, act, n, row, nl, st)
        vrow = self.v_first[0].numel() * self.v_first.element_size()
        vf = cache._v_first.contiguous()
        if to_cache:
            _slot_copy(self.v_first.data_ptr(), 0, vrow, idx, vf.data_ptr(), 0, vrow, None, None, n, vrow, 1, st)
        else:
            _slot_copy(vf.data_ptr(), 0, vrow, None, self.v_first.data_ptr(), 0, vrow, idx, act, n, vrow, 1, st)

    def gather_cache(self, slot_ids, cache=None, *, allow_scratch: bool = False):
        """A batch cache of the slots' state (every layer; rows in slot_ids order)."""
        from .model import NativeRWKV7Cache

        live = [s for s in slot_ids if not (allow_scratch and int(s) == self.scratch_slot)]
        self.check(live)
        if cache is None:
            cache = NativeRWKV7Cache.zeros(self.config, len(slot_ids), self.device, self.dtype)
        if cache.get_batch_size() != len(slot_ids):
            raise ValueError("gather_cache: cache batch differs from the slot count")
        self._batch_copy(cache, list(slot_ids), to_cache=True)
        seen = [self.seen_tokens[int(s)] for s in live]
        cache.seen_tokens = max(seen) if seen else 0
        return cache

    def scatter_cache(self, slot_ids, cache, active=None, *, advance: int = 0) -> None:
        """Commit a batch cache's rows to the slots (only ``active`` rows; the
        scratch slot is never written) and advance their seen_tokens."""
        slot_ids = [int(s) for s in slot_ids]
        active = [1] * len(slot_ids) if active is None else [int(bool(a)) for a in active]
        active = [a if s != self.scratch_slot else 0 for s, a in zip(slot_ids, active)]
        self.check([s for s, a in zip(slot_ids, active) if a])
        self._batch_copy(cache, slot_ids, to_cache=False, active=active)
        for s, a in zip(slot_ids, active):
            if a:
                self.seen_tokens[s] += int(advance)

    # ------------------------------------------------------------ prefix cache
    def fingerprint(self) -> str:
        c = self.config
        key = (LAYOUT_VERSION, c.num_hidden_layers, c.num_heads, c.head_dim, c.hidden_size,
               c.attention_hidden_size, str(self.dtype))
        return hashlib.sha256(repr(key).encode()).hexdigest()

    def snapshot(self, slot: int) -> dict:
        """An immutable host copy of one slot (prefix-state cache entry)."""
        self.check([slot])
        entry = {
            "state": self.state[:, slot].cpu().clone(), "xpa": self.xpa[:, slot].cpu().clone(),
            "xpf": self.xpf[:, slot].cpu().clone(), "v_first": self.v_first[slot].cpu().clone(),
            "seen_tokens": self.seen_tokens[slot], "fingerprint": self.fingerprint(),
        }
        entry["checksum"] = hashlib.sha256(b"".join(entry[k].contiguous().view(torch.uint8).numpy().tobytes()
                                                    for k in ("state", "xpa", "xpf", "v_first"))).hexdigest()
        return entry

    def restore(self, entry: dict, destination_slot: int) -> None:
        """Validate the entry's fingerprint and checksum, then copy it into a live slot."""
        self.check([destination_slot])
        if entry.get("fingerprint") != self.fingerprint():
            raise ValueError("restore: snapshot fingerprint does not match this pool")
        got = hashlib.sha256(b"".join(entry[k].contiguous().view(torch.uint8).numpy().tobytes()
                                      for k in ("state", "xpa", "xpf", "v_first"))).hexdigest()
        if got != entry.get("checksum"):
            raise ValueError("restore: snapshot checksum mismatch")
        d = int(destination_slot)
        self.state[:, d].copy_(entry["state"].to(self.device))
        self.xpa[:, d].copy_(entry["xpa"].to(self.device))
        self.xpf[:, d].copy_(entry["xpf"].to(self.device))
        self.v_first[d].copy_(entry["v_first"].to(self.device))
        self.seen_tokens[d] = int(entry["seen_tokens"])


class PooledDecoder:
    """Graph-bucketed prefill and decode over pool slots (continuous batching)."""

    def __init__(self, model, pool: RWKV7StatePool, buckets=(1, 2, 4, 8, 16, 32, 64), *, use_graph: bool = True):
        self.model = model
        self.pool = pool
        self.buckets = tuple(sorted(int(b) for b in buckets))
        self.use_graph = use_graph
        self._caches: dict[int, object] = {}

    def bucket(self, n: int) -> int:
        for b in self.buckets:
            if b >= n:
                return b
        raise ValueError(f"{n} rows exceed the largest bucket {self.buckets[-1]}")

    def prefill(self, slot_ids, generations, input_ids: torch.Tensor) -> torch.Tensor:
        """Consume ``input_ids [n, T]`` (one row per slot, equal lengths) from
        the slots' current state; returns the last-token logits [n, V]."""
        self.pool.check(slot_ids, generations)
        cache = self.pool.gather_cache(slot_ids)
        out = self.model(input_ids, past_key_values=cache, use_graph=False)
        self.pool.scatter_cache(slot_ids, out.past_key_values, advance=int(input_ids.shape[1]))
        return out.logits[:, -1]

    def step(self, slot_ids, generations, tokens) -> torch.Tensor:
        """One decode token for each slot; returns logits [n, V].  Padding rows
        read the scratch slot and are never committed."""
        self.pool.check(slot_ids, generations)
        n = len(slot_ids)
        b = self.bucket(n)
        rows = [int(s) for s in slot_ids] + [self.pool.scratch_slot] * (b - n)
        active = [1] * n + [0] * (b - n)
        tok = torch.zeros(b, dtype=torch.long, device=self.pool.device)
        tok[:n] = torch.as_tensor(tokens, dtype=torch.long, device=self.pool.device).reshape(-1)
        if self.use_graph:
            runner = self.model.graph_runner(b)
            runner.detach_bound_cache()  # a user cache bound to this bucket keeps its own state
            cache = runner.cache  # the captured graph's own (layer-major) buffers
            self.pool.gather_cache(rows, cache, allow_scratch=True)
            runner.tokens.copy_(tok)
            runner.graph.replay()
            logits = runner.logits
        else:
            cache = self.pool.gather_cache(rows, allow_scratch=True)
            logits = self.model(tok[:, None], past_key_values=cache, use_graph=False).logits[:, -1]
        self.pool.scatter_cache(rows, cache, active, advance=1)
        return logits[:n].clone()  # the runner's buffer is overwritten by the bucket's next replay


__all__ = ["RWKV7StatePool", "PooledDecoder", "LAYOUT_VERSION"]
