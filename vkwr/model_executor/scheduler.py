"""Continuous batching over a WKV slot pool (the reference has no serving code).

Requests arrive with a prompt and a generation budget.  The batcher admits them
into free slots of the recurrent-state pool (resetting the slot's WKV state and
both shift rows), then every step runs one MixedEngine forward over

  * up to `max_decode` sequences that are generating (one token each: the last
    token they produced), and
  * up to `max_prefill_chunks` prompt chunks of at most `chunk` tokens from
    sequences still consuming their prompt (chunks of equal length share one
    prefill group),

within `max_rows` rows in total.  A sequence's first generated token comes from
the logits of its last prompt chunk; each later one from its decode row.
Finished sequences release their slot immediately, so waiting requests are
admitted the next step (256 decode rows + 4 x 512 prefill
rows per step, 2048-slot pool).  The default sampler is greedy (argmax); pass
`sample` to use another, e.g. a ``GpuSampler`` (temperature / top-k / top-p on
the vkwr_sampling kernels).
"""
from collections import deque
from dataclasses import dataclass, field

import torch


@dataclass
class Request:
    prompt: list
    max_new_tokens: int
    rid: int = -1
    slot: int = -1
    pos: int = 0                       # prompt tokens consumed
    output: list = field(default_factory=list)

    @property
    def prefilling(self):
        return self.pos < len(self.prompt)

    @property
    def done(self):
        return len(self.output) >= self.max_new_tokens


class SlotAllocator:
    """Free list over the state pool's slots (FIFO reuse).  Freeing a slot that is out of
    range or not allocated raises RuntimeError, so the slot lists the batcher builds from
    allocated slots are distinct and in range: it checks them on the host and passes
    them to the kernels without a device-side check."""

    def __init__(self, n_slots):
        self.n_slots = n_slots
        self._free = deque(range(n_slots))
        self._used = set()

    def alloc(self):
        if not self._free:
            return None
        slot = self._free.popleft()
        self._used.add(slot)
        return slot

    def free(self, slot):
        if not (0 <= slot < self.n_slots) or slot not in self._used:
            raise RuntimeError(f"slot {slot} is not allocated (pool of {self.n_slots})")
        self._used.remove(slot)
        self._free.append(slot)

    @property
    def available(self):
        return len(self._free)


class ContinuousBatcher:
    def __init__(self, engine, state, max_decode=256, max_prefill_chunks=4, chunk=512, sample=None):
        assert chunk >= 1 and max_decode + chunk <= engine.max_rows
        # every decode row and every chunk's sequence gets a logits row
        assert max_decode + max_prefill_chunks <= engine.max_seqs, (max_decode, max_prefill_chunks, engine.max_seqs)
        self.engine, self.state = engine, state
        self.max_decode, self.max_prefill_chunks, self.chunk = max_decode, max_prefill_chunks, chunk
        self.max_rows = engine.max_rows
        self.slots = SlotAllocator(state.n_slots)
        self.waiting = deque()
        self.running = []
        self.sample = sample or (lambda logits: torch.argmax(logits.float(), dim=-1))
        self.device = engine.model.head.device
        self._next_id = 0
        self._rr = 0  # round-robin start among the decoding sequences
        self.steps = 0
        self.tokens_processed = 0

    def submit(self, prompt, max_new_tokens):
        assert len(prompt) >= 1 and max_new_tokens >= 1
        req = Request(list(prompt), max_new_tokens, rid=self._next_id)
        self._next_id += 1
        self.waiting.append(req)
        return req

    def _reset_slot(self, slot):
        st = self.state
        st.wkv[:, slot].zero_()
        st.att_shift[:, slot].zero_()
        st.ffn_shift[:, slot].zero_()

    def _i32(self, values):
        return torch.tensor(values, dtype=torch.int32).to(self.device, non_blocking=True)

    def _check_slots(self, reqs):
        """Host-side slot-table check of one step (no device sync): every slot allocated,
        each used by one sequence only."""
        slots = [r.slot for r in reqs]
        if len(set(slots)) != len(slots) or any(s not in self.slots._used for s in slots):
            raise RuntimeError(f"invalid slot table for this step: {slots}")

    def step(self):
        """Runs one forward step; returns the requests that finished in it."""
        while self.waiting and self.slots.available:
            req = self.waiting.popleft()
            req.slot = self.slots.alloc()
            self._reset_slot(req.slot)
            self.running.append(req)
        decoding = [r for r in self.running if not r.prefilling]
        if len(decoding) > self.max_decode:
            # more generating sequences than decode rows: rotate, so none starves
            start = self._rr % len(decoding)
            dec = (decoding[start:] + decoding[:start])[: self.max_decode]
            self._rr = start + self.max_decode
        else:
            dec = decoding
        rows = len(dec)
        groups = {}  # chunk length -> requests
        n_chunks = 0
        for r in self.running:
            if not r.prefilling or n_chunks == self.max_prefill_chunks:
                continue
            t = min(self.chunk, len(r.prompt) - r.pos, self.max_rows - rows)
            if t <= 0:
                break
            groups.setdefault(t, []).append(r)
            rows += t
            n_chunks += 1
        if rows == 0:
            return []
        self._check_slots(dec + [r for reqs in groups.values() for r in reqs])
        decode = None
        if dec:
            decode = (self._i32([r.output[-1] for r in dec]), self._i32([r.slot for r in dec]))
        prefill, order = [], []
        for t, reqs in groups.items():
            toks = self._i32([r.prompt[r.pos:r.pos + t] for r in reqs])
            prefill.append((toks, self._i32([r.slot for r in reqs])))
            order.append((t, reqs))
        logits = self.engine.step(self.state, decode=decode, prefill=prefill)
        nxt = self.sample(logits).tolist()
        for i, r in enumerate(dec):
            r.output.append(nxt[i])
        j = len(dec)
        for t, reqs in order:
            for r in reqs:
                r.pos += t
                if not r.prefilling:
                    r.output.append(nxt[j])
                j += 1
        self.steps += 1
        self.tokens_processed += rows
        finished = [r for r in self.running if r.done]
        for r in finished:
            self.slots.free(r.slot)
        self.running = [r for r in self.running if not r.done]
        return finished

    def run(self, max_steps=1 << 30):
        """Steps until every submitted request finished; returns them in completion order."""
        done = []
        while (self.waiting or self.running) and self.steps < max_steps:
            done += self.step()
        return done


__all__ = ["Request", "SlotAllocator", "ContinuousBatcher"]
