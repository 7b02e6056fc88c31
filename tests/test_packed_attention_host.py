"""Host-side routing of PackedAttention on the CPU: which predictor first-step masks count as
the 2x2 causal mask (continuous.py:39-40: zeros with finfo.min above the diagonal; no mask
means causal for two queries, npu_attention.py:17-18), and the bounded cache of results."""
import numpy as np
import torch

from oracle import rope as orope

from qwen3_tts_engine_amd import packed_attention as pa


def causal_mask(dtype, batch=1):
    mask = torch.zeros(batch, 1, 2, 2, dtype=dtype)
    mask[..., 0, 1] = torch.finfo(dtype).min
    return mask


def test_reference_mask_and_no_mask_are_causal():
    for dtype in (torch.bfloat16, torch.float16, torch.float32):
        assert pa._is_causal_pair(causal_mask(dtype), 4)
        assert pa._is_causal_pair(causal_mask(dtype, batch=4), 4)
        mask = causal_mask(dtype)
        mask[..., 0, 1] = float('-inf')
        assert pa._is_causal_pair(mask, 4)
    assert pa._is_causal_pair(None, 4)


def test_other_masks_are_not_causal():
    full = torch.zeros(1, 1, 2, 2, dtype=torch.bfloat16)
    assert not pa._is_causal_pair(full, 4)
    shifted = causal_mask(torch.float32)
    shifted[..., 1, 0] = -5.0
    assert not pa._is_causal_pair(shifted, 4)
    weak = torch.zeros(1, 1, 2, 2)
    weak[..., 0, 1] = -1e30  # large but above finfo.min: a real additive bias, not a mask
    assert not pa._is_causal_pair(weak, 4)
    assert not pa._is_causal_pair(causal_mask(torch.bfloat16, batch=3), 4)  # batch mismatch
    assert not pa._is_causal_pair(torch.zeros(1, 1, 2, 3), 4)
    assert not pa._is_causal_pair(torch.ones(1, 1, 2, 2, dtype=torch.bool), 4)


def test_results_follow_in_place_changes_and_the_cache_is_bounded():
    mask = causal_mask(torch.bfloat16)
    assert pa._is_causal_pair(mask, 4)
    mask.zero_()  # a new tensor version is read again
    assert not pa._is_causal_pair(mask, 4)
    for i in range(3 * pa._CAUSAL_PAIR_LIMIT):
        pa._is_causal_pair(causal_mask(torch.float32) * (1 + i % 2), 4)
    assert len(pa._CAUSAL_PAIR) <= pa._CAUSAL_PAIR_LIMIT


def test_section_axes_follow_the_oracle_selection():
    """The per-dimension axis table PackedAttention gathers with equals the oracle's
    sectioned and interleaved selections (pinned by hand and against transformers)."""
    tables = np.stack([1000.0 * a + np.arange(128.0) for a in range(3)])[:, None, :]
    for sections in ([24, 20, 20], [16, 24, 24], [32, 16, 16]):
        for interleaved in (False, True):
            axes = pa._section_axes(128, sections, interleaved, 'cpu').numpy()
            expected = (orope.mrope_select(tables, sections, interleaved)[0] // 1000).astype(int)
            assert axes.tolist() == expected.tolist()
