"""decode_batch_size of the package against the reference's known answers and invariants
(tests/test_batching.py:6-25 of the reference) and against the oracle's independent search
restatement over every geometry up to a 1024-slot arena.  CPU only."""
import pytest

from oracle import scheduler as osched


def test_reference_known_answers(pkg):
    assert pkg.decode_batch_size(33, 64) == 64
    assert pkg.decode_batch_size(33, 64, 8) == 40
    assert pkg.decode_batch_size(17, 64, 8) == 24


def test_all_active_counts_fit_buckets_without_exceeding_arena(pkg):
    for slots in [1, 2, 4, 8, 16, 32, 64]:
        for step in [0] + [x for x in [1, 2, 4, 8, 16, 32, 64] if x <= slots]:
            for active in range(1, slots + 1):
                batch = pkg.decode_batch_size(active, slots, step)
                assert active <= batch <= slots
                if step and active > step:
                    assert batch % step == 0 and batch - active < step
                else:
                    assert batch & (batch - 1) == 0
                    assert batch == active or batch // 2 < active


def test_matches_oracle_search_everywhere(pkg):
    for slots in [1 << e for e in range(11)]:
        for step in [0] + [1 << e for e in range(11) if (1 << e) <= slots]:
            for active in range(1, slots + 1):
                assert pkg.decode_batch_size(active, slots, step) == osched.decode_batch_size(active, slots, step)


@pytest.mark.parametrize('active,slots,step', [(0, 64, 8), (65, 64, 8), (1, 3, 0), (1, 64, -1),
                                               (1, 64, 3), (1, 8, 16)])
def test_invalid_scheduling_geometry_is_rejected(pkg, active, slots, step):
    with pytest.raises(ValueError):
        pkg.decode_batch_size(active, slots, step)
