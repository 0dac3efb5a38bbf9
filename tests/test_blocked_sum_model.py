"""The arithmetic behind the device sampler's parallel evaluation of a sequential f32 sum
(sample_token_from_logits' sum_e and its inverse-CDF walk, core/sampler.mojo:284-305, and the
running sums of apply_top_p / apply_min_p, :128-147, :175-181), checked on the CPU.

The claim: while acc = fl(acc + t) stays in one binade [2^E, 2^(E+1)), its bit pattern counts ulps
u = 2^(E-23), and for t >= 0, fl(acc + t) = acc + RN(t / u) ulps, unless t / u is exactly halfway
between two integers or the result leaves the binade. So for a block of terms, K_E = sum RN(t / u)
advances the bits exactly whenever acc's bits lie in [first pattern of E, last pattern of E - K_E]
and no term is a halfway case. The model below evaluates sums that way (blocks of 256 and 32
terms, candidate binades from an f64 estimate, a term-by-term fallback) and must reproduce the
plain sequential f32 sum bit for bit, at every block start and at the end, on term sets chosen to
break it: exps, dyadic values with few mantissa bits (many halfway cases), powers of two,
subnormals, zeros and NaN."""
import math

import numpy as np

CHUNK, BLOCK = 256, 32


def seq_prefix(terms):
    """acc after each term, plain sequential f32 (the reference's order)."""
    out = np.empty(len(terms) + 1, np.float32)
    acc = np.float32(0.0)
    out[0] = acc
    with np.errstate(invalid="ignore", over="ignore"):
        for i, t in enumerate(terms):
            acc = np.float32(acc + t)
            out[i + 1] = acc
    return out


def ulps(t, e):
    """RN(t / 2^(e-23)) and the halfway flag; NaN / inf / negative terms are flagged."""
    t = float(t)
    if not (t >= 0.0) or math.isinf(t):
        return 1 << 24, True
    x = t * 2.0 ** (23 - e)  # exact: a power-of-two scale of a 24-bit value
    if x >= 16777216.0:
        return 1 << 24, False
    f = math.floor(x)
    r = x - f
    return int(f) + (1 if r > 0.5 else 0), r == 0.5


def range_of(e, k, half):
    """(lo, span, k) of a block for binade e: bits in [lo, lo + span] advance by k."""
    if e is None or half or k > 0x7FFFFF:
        return 0xFFFFFFFF, 0, 0
    return (e + 127) << 23, 0x7FFFFF - k, k


def step(bits, rng):
    lo, span, k = rng
    if (bits - lo) & 0xFFFFFFFF <= span:
        return True, bits + k
    return False, bits


def bits_of(x):
    return int(np.float32(x).view(np.uint32))


def float_of(b):
    return np.uint32(b).view(np.float32)


def blocked_prefix_at_blocks(terms):
    """The model: the running sum at every chunk start and at the end, by chunk, block and term
    steps."""
    n = len(terms)
    nch = (n + CHUNK - 1) // CHUNK
    csum = [float(np.sum(terms[c * CHUNK:(c + 1) * CHUNK], dtype=np.float64)) for c in range(nch)]
    A, est, starts = 0, 0.0, []
    for c in range(nch):
        starts.append(A)
        e = None
        if 0.0 < est < 1e30:
            cand = math.frexp(est * (1.0 - 1.0 / 64))[1] - 1
            if -100 <= cand <= 100:
                e = cand
        est += csum[c]
        seg = terms[c * CHUNK:(c + 1) * CHUNK]
        blocks = [seg[j:j + BLOCK] for j in range(0, len(seg), BLOCK)]
        per = []
        for blk in blocks:
            row = []
            for x in (0, 1):
                ee = None if e is None else e + x
                ks, hf = 0, False
                for t in blk:
                    if ee is None:
                        break
                    q, h = ulps(t, ee)
                    ks += min(q, 1 << 24)
                    hf |= h
                row.append((min(ks, 1 << 24), hf, ee))
            per.append(row)
        # the chunk's ranges, then its blocks'
        moved = False
        for x in (0, 1):
            ks = min(sum(p[x][0] for p in per), 1 << 24)
            hf = any(p[x][1] for p in per)
            ok, A2 = step(A, range_of(per[0][x][2], ks, hf))
            if ok:
                A, moved = A2, True
                break
        if moved:
            continue
        for bi, blk in enumerate(blocks):
            done = False
            for x in (0, 1):
                ok, A2 = step(A, range_of(per[bi][x][2], per[bi][x][0], per[bi][x][1]))
                if ok:
                    A, done = A2, True
                    break
            if done:
                continue
            a = float_of(A)
            with np.errstate(invalid="ignore", over="ignore"):
                for t in blk:
                    a = np.float32(a + t)
            A = bits_of(a)
    return starts, A


def term_sets(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 3000))
    kind = seed % 7
    if kind == 0:  # exps of f16 logits, as the sampler's
        x = (rng.standard_normal(n) * 2.0).astype(np.float16).astype(np.float32)
        t = np.exp((x - x.max()).astype(np.float64)).astype(np.float32)
    elif kind == 1:  # few mantissa bits: many halfway cases
        t = (rng.integers(0, 4096, n) / 4096.0).astype(np.float32)
    elif kind == 2:  # powers of two
        t = np.ldexp(1.0, -rng.integers(0, 30, n)).astype(np.float32)
    elif kind == 3:  # zeros and small dyadics
        t = np.where(rng.integers(0, 3, n) == 0, 0.0, np.ldexp(rng.integers(0, 256, n), -rng.integers(0, 40, n)))
        t = t.astype(np.float32)
    elif kind == 4:  # down to subnormals
        t = np.ldexp(1.0, -rng.integers(0, 150, n)).astype(np.float32)
    elif kind == 5:  # a NaN among uniform terms
        t = rng.random(n).astype(np.float32)
        t[rng.integers(0, n)] = np.nan
    else:  # probabilities (terms / their sum), as top-p's second pass
        e = np.exp(-30.0 * rng.random(n)).astype(np.float32)
        s = seq_prefix(e)[-1]
        t = (e / s).astype(np.float32)
    return t


def same(a, b):
    return (np.isnan(a) and np.isnan(b)) or a == b


def test_blocked_sum_matches_sequential_sum():
    for seed in range(70):
        t = term_sets(seed)
        ref = seq_prefix(t)
        starts, end = blocked_prefix_at_blocks(t)
        for c, b in enumerate(starts):
            assert same(float_of(b), ref[c * CHUNK]), (seed, c)
        assert same(float_of(end), ref[-1]), seed


def test_blocked_sum_takes_the_integer_steps_on_exps():
    """On the sampler's typical terms most chunks advance in one integer step (the model would be
    pointless otherwise): count the chunks whose start-to-end advance equals their chunk-level
    range's increment."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(40000) * 2.0).astype(np.float16).astype(np.float32)
    t = np.exp((x - x.max()).astype(np.float64)).astype(np.float32)
    ref = seq_prefix(t)
    starts, end = blocked_prefix_at_blocks(t)
    assert same(float_of(end), ref[-1])
    # the bit advance of a chunk that stays in one binade is its ulp count: most chunks do
    same_binade = sum(1 for c in range(len(starts) - 1) if (starts[c] >> 23) == (starts[c + 1] >> 23))
    assert same_binade >= 0.9 * (len(starts) - 1)
