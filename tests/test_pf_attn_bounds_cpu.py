"""The bounds model of the prompt pass's MFMA attention (tests/
pf_attn_bounds.py): every global and LDS access of k_pf_attn_mf stays inside
its buffer, every (prompt row, key position up to its own) pair is covered
by exactly one wave's chunk, and each key's V^T column is the one its MFMA
fragment reads, for one-pass and offset prompts (ragged row counts, passes
ending at the cache's last row), 1, 2, 7 and 8 q heads per kv head; planted
mistakes are reported."""
import pytest

import pf_attn_bounds as pb


@pytest.mark.parametrize("hpk", [1, 7, 8])
@pytest.mark.parametrize("pos0,M,max_ctx", [(0, 1, 1), (0, 2, 64), (0, 37, 64), (0, 256, 256), (0, 256, 4160),
                                            (256, 44, 320), (1000, 64, 1064), (3904, 256, 4160), (63, 33, 96)])
def test_pf_attention_in_bounds_and_covering(hpk, pos0, M, max_ctx):
    r = pb.simulate(2, hpk, max_ctx, pos0, M)
    assert not r.violations, r.violations[:3]
    assert r.checked > 0


def test_pf_attention_row_stride_wider_than_the_heads():
    r = pb.simulate(4, 7, 512, 100, 77, ldx=4 * 7 * 128 + 256)
    assert not r.violations, r.violations[:3]


@pytest.mark.parametrize("mistake", ["row", "perm"])
def test_pf_attention_planted_mistake_is_reported(mistake):
    r = pb.simulate(2, 2, 100, 0, 100, mistake=mistake)
    assert r.violations
