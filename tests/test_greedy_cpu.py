"""decode_greedy_cuda's host logic on the CPU: the chunked loop and its EOS scan against the
reference's loop (bindings_prefill.cpp:1296-1340, restated in oracle/greedy_ref.py), with the
device chain replaced by a stub that replays a fixed greedy sequence.

The restatement is pinned first by known answers worked out by hand from the reference's loop:
the chunk's tail token is emitted but never scanned, a chunk of one step is not scanned at all,
and the final chunk's tail is not emitted."""
import random

import pytest
import torch

from megaqwen_amd.decoder import MegakernelPrefillDecoder
from oracle.greedy_ref import decode_greedy_reference as ref

EOS = 99


def test_reference_loop_known_answers():
    seq = [10, 11, 12, EOS, 13, 14, 15, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25]
    # EOS inside the first chunk: the chunk's tokens before it are kept
    assert ref(seq, 12, [EOS], chunk=8) == ([10, 11, 12], 3, 1)
    # EOS at index 3 = the tail of a 3-step chunk: emitted as the next chunk's first token
    assert ref(seq, 9, [EOS], chunk=3) == ([10, 11, 12, EOS, 13, 14, 15, 16, 17], 9, 0)
    # chunks of one step are never scanned
    assert ref(seq, 6, [EOS], chunk=1) == ([10, 11, 12, EOS, 13, 14], 6, 0)
    # the final chunk's tail (seq[3] for max_new 3) is decoded but not emitted
    assert ref(seq, 3, [EOS], chunk=4) == ([10, 11, 12], 3, 0)
    # index 3 is tokens[1] of the chunk starting at 2 (scanned), not a tail
    assert ref(seq, 8, [EOS], chunk=2) == ([10, 11, 12], 3, 1)
    assert ref(seq, 8, [EOS], chunk=5) == ([10, 11, 12], 3, 1)
    # the first token is never scanned
    assert ref([EOS, 1, 2, 3], 3, [EOS], chunk=4) == ([EOS, 1, 2], 3, 0)
    assert ref(seq, 0, [EOS]) == ([], 0, 0)
    assert ref(seq, 5, [EOS], chunk=0) == ([10, 11, 12], 3, 1)    # chunk <= 0 means 32
    with pytest.raises(RuntimeError):
        ref(seq, 5, [])


class _StubChain(MegakernelPrefillDecoder):
    """decode_greedy_cuda over a fixed greedy sequence: _chain(first, n) returns
    seq[pos .. pos + n] as the device chain would (toks[0] = first)."""

    def __init__(self, seq, vocab=128):
        self._seq = list(seq)
        self.vocab_size = vocab
        self._tok = torch.zeros(2, dtype=torch.int32)
        self._at = 0

    def _chain(self, first_token_id, num_steps):
        assert first_token_id == self._seq[self._at], (first_token_id, self._at)
        toks = torch.tensor(self._seq[self._at:self._at + num_steps + 1], dtype=torch.int32)
        assert toks.numel() == num_steps + 1
        self._at += num_steps
        return toks


def _run(seq, max_new, eos, chunk, **kw):
    out, k, code = _StubChain(seq).decode_greedy_cuda(seq[0], max_new, eos, chunk, **kw)
    return out.tolist(), k, code


def test_decode_greedy_host_loop_matches_reference():
    rng = random.Random(5)
    cases = 0
    for _ in range(400):
        n = rng.randint(1, 90)
        seq = [rng.randrange(0, 12) for _ in range(n + 1)]
        eos = [rng.randrange(0, 12) for _ in range(rng.randint(1, 2))]
        for chunk in (1, 2, 3, 7, 8, 32, 0):
            assert _run(seq, n, eos, chunk) == ref(seq, n, eos, chunk), (seq, n, eos, chunk)
            cases += 1
    # an EOS exactly at every chunk tail position of a long chain, then on the final tail
    for chunk in (4, 8, 16):
        for j in range(1, 41):
            seq = [1] * 41
            seq[j] = EOS
            assert _run(seq, 40, [EOS], chunk) == ref(seq, 40, [EOS], chunk), (chunk, j)
    assert cases > 2000


def test_scan_chunk_tail_gives_the_prefix_before_the_first_eos():
    """The opt-in scan of the chunk tails: the result is the greedy sequence up to, not
    including, its first EOS after the first token (or max_new tokens without one)."""
    rng = random.Random(9)
    for _ in range(300):
        n = rng.randint(1, 70)
        seq = [rng.randrange(0, 10) for _ in range(n + 1)]
        eos = [rng.randrange(0, 10)]
        js = [j for j in range(1, n + 1) if seq[j] in eos]
        want = (seq[:js[0]], js[0], 1) if js else (seq[:n], n, 0)
        for chunk in (1, 3, 8, 32):
            assert _run(seq, n, eos, chunk, scan_chunk_tail=True) == want, (seq, eos, chunk)
