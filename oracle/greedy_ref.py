"""CPU restatement of the reference's chunked greedy loop.  TEST INFRASTRUCTURE ONLY.

Only `tests/` may import this module, as the checker of `decode_greedy_cuda`'s host logic.

`decode_greedy_reference` follows MegakernelPrefillDecoder::decode_greedy_cuda with the default
"coop" decode backend, csrc/megakernel/bindings_prefill.cpp:1159-1182 (argument handling) and
:1296-1340 (the loop), given the greedy continuation `seq` of the first token (seq[0] = first
token, seq[i + 1] = the token decoded from seq[i]): per chunk of `steps` decode steps,
tokens[0..steps] = seq[gen .. gen + steps]; tokens[0..steps-1] are appended to the output
(:1307-1308); tokens[1..steps-1] are scanned for the first EOS id, and not at all when steps == 1
(:1310-1321); an EOS at scanned index i keeps i + 1 tokens of the chunk and stops with code 1
(:1329-1333); otherwise tokens[steps] is the next chunk's tokens[0] (:1336-1338).
"""
from __future__ import annotations


def decode_greedy_reference(seq, max_new_tokens: int, eos_ids, chunk: int = 32,
                            with_steps: bool = False):
    """(tokens list, count, stop_code) of the reference loop over the greedy sequence `seq`
    (which must hold at least max_new_tokens + 1 entries); with `with_steps`, also the number
    of decode steps run, by which the reference advances position_ (:1324)."""
    max_new = int(max_new_tokens)
    if max_new <= 0:
        return ([], 0, 0, 0) if with_steps else ([], 0, 0)
    if chunk <= 0:
        chunk = 32
    eos = set(int(e) for e in eos_ids)
    if not eos:
        raise RuntimeError("eos_ids must be a non-empty int32 tensor")
    out: list[int] = []
    gen = 0
    while gen < max_new:
        steps = min(chunk, max_new - gen)
        tokens = [int(t) for t in seq[gen:gen + steps + 1]]
        assert len(tokens) == steps + 1, "seq is shorter than the decoded chain"
        out.extend(tokens[:steps])
        stop_pos = -1
        if steps > 1:
            for i, t in enumerate(tokens[1:steps]):
                if t in eos:
                    stop_pos = i + 1
                    break
        if stop_pos >= 0:
            decoded = gen + steps
            gen += stop_pos
            return (out[:gen], gen, 1, decoded) if with_steps else (out[:gen], gen, 1)
        gen += steps
    return (out[:gen], gen, 0, gen) if with_steps else (out[:gen], gen, 0)
