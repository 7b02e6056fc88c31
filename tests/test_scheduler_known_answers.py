"""Known-answer traces of the continuous-batching tick, worked out by hand from the reference.

Every expected value below was derived on paper from ContinuousModel.tick
(qwen3_tts_engine/continuous.py:541-657), admit_batch (:425-473), ensure_capacity (:353-363)
and decode_batch_size (batching.py:4-11), not produced by running either scheduler.  The same
traces run through the oracle's restatement (oracle/scheduler.py) and the package's
SlotScheduler, so a wrong rule in either one fails here:

* cancellations are applied before admissions, in reverse slot order, and each one moves the
  last slot into the freed index (:545-555);
* a new request takes slot ``len(states)`` (:469-472) at position = prompt length;
* growth happens when a requirement reaches the capacity, to ``max(2C, 2**bit_length(req))``
  (:353-363): at admission for the longest prompt (:460) and before decode for the largest
  position (:572);
* the graph batch pads with position-0 rows (:571, :602);
* with bucket_kv the context is ``min(C, max(64, 2**bit_length(max_pos)))`` (:605-606);
* after decode every request gains one frame and one position and retires once
  ``frames >= max_new_tokens - 1`` (:628-642), finished requests leave in reverse slot order
  with last-into-freed moves (:645-656).

Each tick is written as (submissions, cancelled, expected record or None, expected retired
identifiers in retirement order, expected operations)."""
import pytest

from oracle import scheduler as osched


class _Package:
    """The package scheduler behind the oracle's tick contract."""

    def __init__(self, *args, **kwargs):
        from qwen3_tts_engine_amd.scheduler import SlotScheduler
        self.inner = SlotScheduler(*args, **kwargs)

    @property
    def ops(self):
        return self.inner.ops

    def tick(self, submissions=(), cancelled=()):
        batch, done = self.inner.tick(submissions, cancelled)
        if batch is None:
            return None, done
        return {'batch': batch.batch, 'context': batch.context, 'positions': batch.positions,
                'slots': batch.identifiers, 'capacity': batch.capacity}, done


def _rec(batch, context, positions, slots, capacity):
    return {'batch': batch, 'context': context, 'positions': positions, 'slots': slots,
            'capacity': capacity}


def _run(make, ticks):
    scheduler = make()
    for i, (subs, cancelled, record, done, ops) in enumerate(ticks):
        got, finished = scheduler.tick(subs, cancelled)
        assert got == record, f"tick {i + 1}: record {got} != {record}"
        assert finished == done, f"tick {i + 1}: retired {finished} != {done}"
        assert list(scheduler.ops) == ops, f"tick {i + 1}: ops {scheduler.ops} != {ops}"


def _both(args, kwargs, ticks):
    _run(lambda: osched.ReferenceScheduler(*args, **kwargs), ticks)
    _run(lambda: _Package(*args, **kwargs), ticks)


@pytest.fixture
def both(pkg):
    return _both


# -- retirement exactly at frames == max_new_tokens - 1 (continuous.py:628, 638) ----------------

def test_retirement_at_frames_equal_limit_minus_one(both):
    """Limits 3, 2 and 1: after the first decode frames = 1, so the limit-2 and limit-1
    requests retire at once (1 >= 1, 1 >= 0) and the limit-3 one only after the second
    decode (2 >= 2).  Both leave in reverse slot order; neither needs a move, because
    slot 2 is the last slot and, once it is gone, so is slot 1."""
    ticks = [
        ([(10, 5, 3), (11, 7, 2), (12, 9, 1)], (),
         _rec(4, 512, [5, 7, 9, 0], [10, 11, 12], 512), [12, 11],
         [('load', 0, 10, 5), ('load', 1, 11, 7), ('load', 2, 12, 9), ('decode', 4, 512)]),
        ((), (), _rec(1, 512, [6], [10], 512), [10], [('decode', 1, 512)]),
        ((), (), None, [], []),
    ]
    both((4, 512), {}, ticks)


# -- cancellation before admission, reverse order (continuous.py:545-561) -----------------------

def test_cancel_and_admit_in_one_tick(both):
    """Tick 2 cancels slot 0 and admits request 3 in the same tick: the cancellation moves
    the last slot (request 2) into slot 0 first, then request 3 takes slot 2.  Tick 3
    cancels the last slot (no move).  Tick 5 cancels slots 0 and 2: slot 2 first (last slot
    3 moves into it), then slot 0 (the new last slot, 2, moves into it)."""
    ticks = [
        ([(0, 10, 100), (1, 20, 100), (2, 30, 100)], (),
         _rec(4, 512, [10, 20, 30, 0], [0, 1, 2], 512), [],
         [('load', 0, 0, 10), ('load', 1, 1, 20), ('load', 2, 2, 30), ('decode', 4, 512)]),
        ([(3, 40, 100)], (0,),
         _rec(4, 512, [31, 21, 40, 0], [2, 1, 3], 512), [],
         [('move', 2, 0), ('load', 2, 3, 40), ('decode', 4, 512)]),
        ((), (3,), _rec(2, 512, [32, 22], [2, 1], 512), [], [('decode', 2, 512)]),
        ([(4, 50, 100), (5, 60, 100)], (),
         _rec(4, 512, [33, 23, 50, 60], [2, 1, 4, 5], 512), [],
         [('load', 2, 4, 50), ('load', 3, 5, 60), ('decode', 4, 512)]),
        ((), (2, 4), _rec(2, 512, [61, 24], [5, 1], 512), [],
         [('move', 3, 2), ('move', 2, 0), ('decode', 2, 512)]),
    ]
    both((8, 512), {}, ticks)


# -- two finishes in one tick: reverse-order last-into-freed moves (continuous.py:645-656) ------

def test_two_finishes_compact_in_reverse_order(both):
    """Requests 1 and 3 (limit 3) finish after the second decode.  Slot 3 goes first: slot 4
    (request 4) moves into it; then slot 1: the new last slot 3 (request 4 again) moves into
    it, leaving [0, 4, 2].  The retired identifiers come out as [3, 1]."""
    ticks = [
        ([(0, 10, 100), (1, 11, 3), (2, 12, 100), (3, 13, 3), (4, 14, 100)], (),
         _rec(8, 512, [10, 11, 12, 13, 14, 0, 0, 0], [0, 1, 2, 3, 4], 512), [],
         [('load', 0, 0, 10), ('load', 1, 1, 11), ('load', 2, 2, 12), ('load', 3, 3, 13),
          ('load', 4, 4, 14), ('decode', 8, 512)]),
        ((), (), _rec(8, 512, [11, 12, 13, 14, 15, 0, 0, 0], [0, 1, 2, 3, 4], 512), [3, 1],
         [('decode', 8, 512), ('move', 4, 3), ('move', 3, 1)]),
        ((), (), _rec(4, 512, [12, 16, 14, 0], [0, 4, 2], 512), [], [('decode', 4, 512)]),
    ]
    both((8, 512), {}, ticks)


def test_finish_of_the_last_slot_needs_no_move(both):
    """Slots 0 and 2 finish together: slot 2 is the last slot (popped, no move), then slot 1
    moves into slot 0."""
    ticks = [
        ([(7, 3, 2), (8, 4, 100), (9, 5, 2)], (),
         _rec(4, 512, [3, 4, 5, 0], [7, 8, 9], 512), [9, 7],
         [('load', 0, 7, 3), ('load', 1, 8, 4), ('load', 2, 9, 5), ('decode', 4, 512),
          ('move', 1, 0)]),
        ((), (), _rec(1, 512, [5], [8], 512), [], [('decode', 1, 512)]),
    ]
    both((4, 512), {}, ticks)


# -- growth when a requirement reaches the capacity (continuous.py:353-363, 460, 572) ----------

def test_growth_when_position_reaches_capacity(both):
    """Capacity 16, prompt 10: decodes at positions 10 ... 15 fit; before the decode at
    position 16 the capacity doubles to max(32, 2**5) = 32.  A 32-token prompt then needs
    max(64, 2**6) = 64 at admission (32 < 32 is false)."""
    ticks = [([(0, 10, 100)], (), _rec(1, 16, [10], [0], 16), [],
              [('load', 0, 0, 10), ('decode', 1, 16)])]
    for position in range(11, 16):
        ticks.append(((), (), _rec(1, 16, [position], [0], 16), [], [('decode', 1, 16)]))
    ticks.append(((), (), _rec(1, 32, [16], [0], 32), [], [('grow', 16, 32), ('decode', 1, 32)]))
    ticks.append(([(1, 32, 100)], (), _rec(2, 64, [17, 32], [0, 1], 64), [],
                  [('grow', 32, 64), ('load', 1, 1, 32), ('decode', 2, 64)]))
    both((2, 16), {}, ticks)


def test_admission_growth_skips_to_the_bit_length(both):
    """A 33-token prompt in a 16-row arena: max(2 * 16, 2**bit_length(33) = 64) = 64."""
    both((2, 16), {}, [([(0, 33, 100)], (), _rec(1, 64, [33], [0], 64), [],
                        [('grow', 16, 64), ('load', 0, 0, 33), ('decode', 1, 64)])])


# -- bucket_kv context (continuous.py:605-606) ---------------------------------------------------

def test_bucket_kv_context_boundaries(both):
    """Largest position 63 -> context 64; 64 -> 128; 127 -> 128; 128 -> 256; a position
    equal to the capacity grows the arena first and the context follows it."""
    ticks = [
        ([(0, 63, 1000)], (), _rec(1, 64, [63], [0], 512), [], [('load', 0, 0, 63), ('decode', 1, 64)]),
        ((), (), _rec(1, 128, [64], [0], 512), [], [('decode', 1, 128)]),
        ([(1, 127, 1000)], (), _rec(2, 128, [65, 127], [0, 1], 512), [],
         [('load', 1, 1, 127), ('decode', 2, 128)]),
        ((), (), _rec(2, 256, [66, 128], [0, 1], 512), [], [('decode', 2, 256)]),
        ([(2, 511, 1000)], (), _rec(4, 512, [67, 129, 511, 0], [0, 1, 2], 512), [],
         [('load', 2, 2, 511), ('decode', 4, 512)]),
        ((), (), _rec(4, 1024, [68, 130, 512, 0], [0, 1, 2], 1024), [],
         [('grow', 512, 1024), ('decode', 4, 1024)]),
    ]
    both((4, 512), {'bucket_kv': True}, ticks)


def test_bucket_kv_short_context_floor(both):
    """A one-token prompt still attends a 64-key context (the floor)."""
    ticks = [([(0, 1, 1000)], (), _rec(1, 64, [1], [0], 512), [], [('load', 0, 0, 1), ('decode', 1, 64)])]
    both((2, 512), {'bucket_kv': True}, ticks)


# -- graph batch with a bucket step (batching.py:4-11, continuous.py:571, 602) ------------------

def test_bucket_step_pads_with_position_zero_rows(both):
    """Step 2 in an 8-slot arena: 3 requests -> batch 4 (one padded row), 5 -> 6."""
    ticks = [
        ([(0, 9, 100), (1, 8, 100), (2, 7, 100)], (), _rec(4, 512, [9, 8, 7, 0], [0, 1, 2], 512), [],
         [('load', 0, 0, 9), ('load', 1, 1, 8), ('load', 2, 2, 7), ('decode', 4, 512)]),
        ([(3, 6, 100), (4, 5, 100)], (), _rec(6, 512, [10, 9, 8, 6, 5, 0], [0, 1, 2, 3, 4], 512), [],
         [('load', 3, 3, 6), ('load', 4, 4, 5), ('decode', 6, 512)]),
    ]
    both((8, 512), {'decode_bucket_step': 2}, ticks)
