"""Launch-plan choices of the runtime that lossless speculation relies on,
checked without a GPU: everything that changes a row's arithmetic must be
the same for the plain and the speculative state of one batch."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "dryft-challenge_amd"))


@pytest.mark.parametrize("batch", list(range(1, 65)))
@pytest.mark.parametrize("group", [1, 2, 4, 5, 8, 16])
def test_attention_waves_fit_every_state_of_a_batch(batch, group):
    from engine import spec_k
    from qdec.runtime import attn_waves, max_rows_per_seq
    waves = attn_waves(batch)
    assert waves in (4, 8)

    def max_t(requested):  # DecodeState's clamp
        return max_rows_per_seq(batch, requested, group)

    k = spec_k(batch, group)
    plain, spec = max_t(16), max_t(k + 1 if k else 16)
    if waves == 8:  # the 8-wave body takes at most 8 rows per sequence
        assert plain <= 8 and spec <= 8
    # query rows per kv head within what the attention takes (qdec_attn)
    assert plain * group <= (32 if waves == 8 else 64) and spec * group <= (32 if waves == 8 else 64)
    assert k + 1 <= max_t(16) or k == 0
    # verify rows of a speculative state stay on the one-M-tile GEMM path
    assert batch * (k + 1) <= 16 or k == 0


def test_lm_head_grouping_divides_the_vocab():
    from qdec.checkpoint import qwen3_config
    from qdec.runtime import LM_TILES_BATCHED, role_plan
    vocab, hidden = qwen3_config()["vocab_size"], qwen3_config()["hidden_size"]
    assert (vocab // 16) % LM_TILES_BATCHED == 0
    assert (vocab // 16) % role_plan(vocab, hidden, "lm")[2] == 0
