"""Pins for oracle.rng: the MT19937 / legacy-randint / random() restatement against numpy's
RandomState (the generator brainstate/nn/_event_fixedprob.py:163-168,186 draws from), and
Philox4x32-10 against the Random123 known-answer vectors."""
import numpy as np
import pytest

from oracle import rng


@pytest.mark.parametrize('seed', [0, 1, 42, 2 ** 32 - 1])
def test_seeding_and_raw_words_equal_numpy(seed):
    ref = np.random.RandomState(seed)
    key = ref.get_state()[1]
    g = rng.MT19937(seed)
    np.testing.assert_array_equal(g.key, key)
    np.testing.assert_array_equal(g.words(3000), ref.randint(0, 2 ** 32, 3000, dtype=np.uint32))


@pytest.mark.parametrize('seed,n_pre,k,n_post', [(1, 300, 80, 4000), (7, 50, 13, 1024),
                                                 (3, 40, 9, 1025), (9, 20, 5, 2),
                                                 (11, 10, 6, 1), (5, 100, 100, 1_000_000),
                                                 (2, 64, 7, 2 ** 31 - 1)])
def test_randint_then_random_equal_numpy(seed, n_pre, k, n_post):
    """Masked rejection (mask = smallest 2^j - 1 >= n_post - 1) and the random() draws that
    continue the stream, as FixedNumConn with afferent_ratio < 1 takes them."""
    ref = np.random.RandomState(seed)
    want_idx = ref.randint(0, n_post, size=(n_pre, k))
    want_u = ref.random(n_pre)
    g = rng.MT19937(seed)
    np.testing.assert_array_equal(g.randint(n_post, (n_pre, k)), want_idx)
    np.testing.assert_array_equal(g.random(n_pre), want_u)


# Random123 known-answer vectors for Philox4x32-10 (counter, key -> output)
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff,) * 4, (0xffffffff, 0xffffffff), (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
]


@pytest.mark.parametrize('ctr,key,out', KAT)
def test_philox_known_answers(ctr, key, out):
    got = rng.philox4x32(np.array(ctr, np.uint32), (np.uint32(key[0]), np.uint32(key[1])))
    assert [int(x) for x in got] == list(out)


def test_unique_rows_properties():
    """Distinct, in range, and (chi-square) uniform over the targets."""
    out = rng.unique_rows(123, 200, 30, 40)
    assert out.min() >= 0 and out.max() < 40
    assert all(len(set(r)) == 30 for r in out.tolist())
    counts = np.bincount(out.ravel(), minlength=40)
    exp = out.size / 40
    chi2 = ((counts - exp) ** 2 / exp).sum()
    assert chi2 < 80   # 39 degrees of freedom, p ~ 1e-4
