"""Integer state of the reference's continuous-batching scheduler, restated.

Follows ContinuousModel (continuous.py): tick (:541-657), admit_batch (:425-473),
ensure_capacity (:353-363) and decode_batch_size (batching.py:4-11).  Only the integer
state is kept: request order in slots, positions, frames, arena capacity, graph batch and
context; device work is recorded as an ordered list of operations.
"""
from dataclasses import dataclass

import numpy as np


def decode_batch_size(active, max_slots, step=0):
    """batching.py:4-11, restated as a search: the smallest admissible bucket that holds
    ``active`` requests.  Admissible buckets are the powers of two up to the step (all of
    them without a step) and then the multiples of the step; both rules require a
    power-of-two arena and a power-of-two step no larger than it."""
    def pow2(n):
        return n > 0 and (n & (n - 1)) == 0
    if not pow2(max_slots) or active < 1 or active > max_slots:
        raise ValueError('Active count must fit a positive power-of-two slot arena')
    if step < 0 or (step > 0 and (not pow2(step) or step > max_slots)):
        raise ValueError('Decode bucket step must be zero or a power of two within the arena')
    limit = step if step else max_slots
    candidates = [1 << e for e in range(max_slots.bit_length()) if (1 << e) <= limit]
    if step:
        candidates += list(range(2 * step, max_slots + 1, step))
    return min(c for c in candidates if c >= active)


@dataclass
class State:
    identifier: int
    position: int
    max_new_tokens: int
    frames: int = 0


class ReferenceScheduler:
    """Integer restatement of ContinuousModel's slot bookkeeping."""

    def __init__(self, max_slots, initial_capacity=512, decode_bucket_step=0, bucket_kv=False):
        if max_slots < 1 or max_slots & (max_slots - 1):
            raise ValueError('Continuous slot count must be a positive power of two')
        decode_batch_size(1, max_slots, decode_bucket_step)
        self.max_slots = max_slots
        self.capacity = initial_capacity
        self.step = decode_bucket_step
        self.bucket_kv = bucket_kv
        self.states = []
        self.ops = []

    def ensure_capacity(self, required):                      # continuous.py:353-363
        if required < self.capacity:
            return
        new = max(self.capacity * 2, 1 << required.bit_length())
        self.ops.append(('grow', self.capacity, new))
        self.capacity = new

    def _remove(self, index):                                  # continuous.py:547-555, 648-656
        last = len(self.states) - 1
        if last != index:
            self.ops.append(('move', last, index))
            self.states[index] = self.states[last]
        self.states.pop()

    def tick(self, submissions=(), cancelled=()):
        """submissions: [(identifier, prompt_length, max_new_tokens)].  Returns the
        decode record (batch, context, positions) or None, plus finished identifiers."""
        self.ops = []
        cancelled = set(cancelled)
        for index in reversed(range(len(self.states))):
            if self.states[index].identifier in cancelled:
                self._remove(index)
        if submissions:                                        # admit_batch
            if len(self.states) + len(submissions) > self.max_slots:
                raise ValueError('Insufficient continuous request slots')
            self.ensure_capacity(max(length for _, length, _ in submissions))
            for identifier, length, limit in submissions:
                self.ops.append(('load', len(self.states), identifier, length))
                self.states.append(State(identifier, length, limit))
        if not self.states:
            return None, []
        count = len(self.states)
        batch = decode_batch_size(count, self.max_slots, self.step)
        self.ensure_capacity(max(s.position for s in self.states))
        positions = [s.position for s in self.states] + [0] * (batch - count)
        required = max(s.position for s in self.states) + 1
        context = (min(self.capacity, max(64, 1 << (required - 1).bit_length()))
                   if self.bucket_kv else self.capacity)
        record = {'batch': batch, 'context': context, 'positions': positions,
                  'slots': [s.identifier for s in self.states], 'capacity': self.capacity}
        self.ops.append(('decode', batch, context))
        finished = []
        for index, state in enumerate(self.states):
            state.frames += 1
            state.position += 1
            if state.frames >= state.max_new_tokens - 1:       # continuous.py:638
                finished.append(index)
        done = []
        for index in reversed(finished):
            done.append(self.states[index].identifier)
            self._remove(index)
        return record, done


def make_trace(seed=0, iterations=200, mean_arrivals=2.0, prompt=(32, 512), lengths=(200, 2000),
               cancel_rate=0.0):
    """Seeded arrivals for the mixed trace: per iteration a list of
    (identifier, prompt_length, max_new_tokens) and a cancellation draw per iteration."""
    rng = np.random.default_rng(seed)
    arrivals, cancels, identifier = [], [], 0
    for _ in range(iterations):
        batch = []
        for _ in range(int(rng.poisson(mean_arrivals))):
            batch.append((identifier, int(rng.integers(prompt[0], prompt[1] + 1)),
                          int(rng.integers(lengths[0], lengths[1] + 1))))
            identifier += 1
        arrivals.append(batch)
        cancels.append(float(rng.random()) if cancel_rate > 0 else 1.0)
    return {'arrivals': arrivals, 'cancels': cancels, 'cancel_rate': cancel_rate}


def drive(scheduler, trace, max_slots):
    """FIFO admission of the trace into ``scheduler`` (any object with the tick contract):
    every iteration submits as many queued requests as there are free slots, and with
    probability cancel_rate cancels the oldest active request.  Returns the per-iteration
    records (decode record, finished identifiers, device ops)."""
    queue, records, active = [], [], []
    for step, batch in enumerate(trace['arrivals']):
        queue.extend(batch)
        cancelled = []
        if trace['cancel_rate'] > 0 and active and trace['cancels'][step] < trace['cancel_rate']:
            cancelled = [active[0]]
        free = max_slots - (len(active) - len(cancelled))
        submissions, queue = queue[:free], queue[free:]
        record, finished = scheduler.tick(submissions, cancelled)
        active = [i for i in active if i not in cancelled and i not in finished]
        active.extend(i for i, _, _ in submissions if i not in finished)
        records.append((record, sorted(finished), list(getattr(scheduler, 'ops', []))))
    return records
