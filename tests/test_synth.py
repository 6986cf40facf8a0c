"""The seeded input generator (google-classic_amd/csrc/synth.c)."""
import numpy as np


def test_deterministic_and_seed_sensitive(synth):
    a = synth.blocks(2, 8, 4096, seed=1)
    assert np.array_equal(a, synth.blocks(2, 8, 4096, seed=1))
    assert not np.array_equal(a, synth.blocks(2, 8, 4096, seed=2))
    x = synth.normal(1000, seed=5)
    assert np.array_equal(x, synth.normal(1000, seed=5))


def test_blocks_are_independent_of_the_tensor_size(synth):
    """block i depends only on (seed, i): a prefix is the same in a bigger tensor."""
    small = synth.blocks(8, 1, 32 * 10, seed=9)
    big = synth.blocks(8, 1, 32 * 1000, seed=9)
    assert np.array_equal(small, big[: small.size])


def test_f16_rne_matches_numpy(synth):
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(5000) * 0.01, rng.standard_normal(2000) * 1e-6,
                         [0.0, 65504.0, 65520.0, 2 ** -25, 2 ** -24]]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal([synth.f32_to_f16_bits(float(v)) for v in xs], want)


def test_value_ranges_follow_the_configs(synth):
    q8 = synth.blocks(8, 64, 4096, seed=3).reshape(-1, 34)
    d8 = q8[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float64)
    qs = q8[:, 2:].view(np.int8)
    assert qs.min() >= -127 and qs.max() <= 127 and qs.min() == -127 and qs.max() == 127
    assert abs(np.mean(d8) - 0.01 * np.sqrt(2 / np.pi)) < 2e-4        # E|N(0,1)| * 0.01
    q4 = synth.blocks(2, 64, 4096, seed=4).reshape(-1, 18)
    nib = np.concatenate([q4[:, 2:] & 15, q4[:, 2:] >> 4]).ravel()
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.9 * counts.mean()                          # uniform nibbles
    d4 = q4[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float64)
    assert abs(np.mean(d4) - 0.02 * np.sqrt(2 / np.pi)) < 4e-4
    x = synth.normal(200000, seed=6)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01


def test_tensor_seeds_are_distinct(synth):
    seeds = {synth.tensor_seed(20251201, c, l, m) for c in range(5) for l in range(32) for m in range(8)}
    assert len(seeds) == 5 * 32 * 8
