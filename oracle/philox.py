"""Philox-4x64-10 counter-based RNG, restated from Salmon et al., "Parallel Random Numbers:
As Easy as 1, 2, 3" (SC'11), in exact Python integer arithmetic.

TEST INFRASTRUCTURE ONLY. Nothing in the product package imports this module; it is the
checker for the HIP sampler (``qtts_philox4x64`` in the device code).

Why a counter-based RNG: the reference samples with ``torch.multinomial``
(/root/reference/qwentts_turbo/generator.py:206-207), whose stream is not reproducible across
devices, so no sampled token of the reference can be reproduced. The build defines the sampler
as Gumbel-max over the same filtered logits (same distribution as softmax+multinomial, see
``oracle.qtts_oracle.sample_token``) with the noise drawn from Philox-4x64-10, so that the
kernel and this oracle consume identical random numbers.

Pinning: ``philox4x64_10`` is checked against ``numpy.random.Philox`` (a library known-answer
source in this container) in ``tests/test_oracle_philox.py``. numpy increments the 256-bit
counter *before* each block, so ``numpy.random.Philox(counter=c, key=k).random_raw(4)`` equals
``philox4x64_10(c + 1, k)``.
"""

M0 = 0xD2E7470EE14C6C93
M1 = 0xCA5A826395121157
W0 = 0x9E3779B97F4A7C15
W1 = 0xBB67AE8584CAA73B
MASK = (1 << 64) - 1


def _round(ctr, key):
    p0 = M0 * ctr[0]
    p1 = M1 * ctr[2]
    hi0, lo0 = p0 >> 64, p0 & MASK
    hi1, lo1 = p1 >> 64, p1 & MASK
    return [hi1 ^ ctr[1] ^ key[0], lo1, hi0 ^ ctr[3] ^ key[1], lo0]


def philox4x64_10(ctr, key):
    """Return the four 64-bit output words for a 4-word counter and 2-word key."""
    c = [int(x) & MASK for x in ctr]
    k = [int(x) & MASK for x in key]
    for r in range(10):
        if r:
            k = [(k[0] + W0) & MASK, (k[1] + W1) & MASK]
        c = _round(c, k)
    return c


def uniform_from_word(w):
    """Map a 64-bit word to a double in the open interval (0, 1): ((w >> 12) + 0.5) * 2**-52.

    The top 52 bits plus one half fit a double's 53-bit significand exactly, so no word maps
    to 0 or 1 (with 53 bits, (2**53 - 1) + 0.5 would round up to 2**53 and give u = 1)."""
    return ((int(w) >> 12) + 0.5) * (1.0 / 4503599627370496.0)


# Sampler stream layout shared with the device code: one Philox block per 4 vocabulary ids.
#   key     = (seed, 0x5154545341464D50)            # "QTTSAFMP" tag in the high key word
#   counter = (vocab_id // 4, frame_step, group, 0)  # group 0 = backbone g0, 1..15 = CP heads
#   word    = vocab_id % 4
KEY_TAG = 0x5154545341464D50


def sampler_uniform(seed, frame_step, group, vocab_id):
    words = philox4x64_10([vocab_id // 4, frame_step, group, 0], [seed, KEY_TAG])
    return uniform_from_word(words[vocab_id % 4])
