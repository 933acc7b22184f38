"""The bounds model of the decode attention kernel (tests/attn_bounds.py):
every global and LDS access of k_attn stays inside its buffer at every
context length of small caches, at sampled lengths of the 7B session's
(4160 positions, where splits take two chunks), for 1..8 query heads per kv
head, with 4 and 8 waves per workgroup and 1 to 3 chunks per split at
least; a planted unclamped index is reported."""
import pytest

import attn_bounds as ab


@pytest.mark.parametrize("waves,min_cps", [(4, 1), (8, 1), (4, 2), (8, 3)])
@pytest.mark.parametrize("hpk", [1, 2, 7, 8])
def test_every_context_of_small_caches_in_bounds(hpk, waves, min_cps):
    n = 0
    for max_ctx in (1, 63, 64, 65, 130, 520):
        for T in range(1, max_ctx + 1, 1 if max_ctx <= 130 else 7):
            r = ab.simulate(2, hpk, max_ctx, T, waves=waves, min_cps=min_cps)
            assert not r.violations, (hpk, max_ctx, T, r.violations)
            n += r.checked
    assert n > 100_000


@pytest.mark.parametrize("waves,min_cps", [(4, 1), (8, 1), (4, 2)])
def test_seven_b_session_lengths_in_bounds(waves, min_cps):
    for T in (1, 64, 65, 448, 449, 512, 513, 516, 2048, 2049, 4095, 4096, 4097, 4100, 4160):
        r = ab.simulate(4, 7, 4160, T, waves=waves, min_cps=min_cps)
        assert not r.violations, (T, r.violations)


@pytest.mark.parametrize("mistake", ["row", "qhead"])
def test_planted_mistake_is_reported(mistake):
    found = any(ab.simulate(2, 7, 600, T, mistake).violations for T in (40, 300, 600))
    assert found
