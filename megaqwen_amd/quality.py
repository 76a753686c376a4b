"""Quality harness: KL divergence, perplexity and argmax agreement of the decoder's logits against
reference logits (experiments/framework_bench/quality_metrics.py:33-238).

The decoder flow is get_megakernel_logits (quality_metrics.py:170-238): reset, feed every prompt
token but the last through decode, take the last position's fp32 logits
(`decode_step_with_logits`, the reference's `decode_ldg_with_logits`) and compare them with the
reference model's last-position logits: KL(P_ref || P_test) and argmax agreement, averaged over
the prompts.

Reference logits are supplied by the caller as tensors (one fp32 [vocab] row per prompt).  In a
real run they come from HuggingFace's Qwen3ForCausalLM on the same local checkpoint (`main`,
quality_metrics.py:99-144); this module needs no model code of its own.
"""
from __future__ import annotations

import argparse
import dataclasses
import sys
from typing import Iterable, List, Optional, Sequence

import torch
import torch.nn.functional as F

# quality_metrics.py:24-30
TEST_PROMPTS = [
    "The quick brown fox jumps over the lazy dog.",
    "In machine learning, gradient descent is",
    "The capital of France is",
    "Write a function to compute fibonacci numbers:",
    "The meaning of life is",
]


@dataclasses.dataclass
class QualityResult:
    """quality_metrics.py:33-40."""
    name: str
    supported: bool
    kl_div: Optional[float]
    perplexity: Optional[float]
    argmax_match: Optional[float]
    error: Optional[str] = None


def _format_float(value: Optional[float], precision: int = 6) -> str:
    return "n/a" if value is None else f"{value:.{precision}f}"


def format_markdown_table(results: Iterable[QualityResult]) -> str:
    """The results table of quality_metrics.py:55-67."""
    lines = ["| Framework | KL Divergence | Perplexity | Argmax Match | Status |",
             "|---|---|---|---|---|"]
    for r in results:
        status = "ok" if r.supported else (r.error or "skipped")
        am = f"{r.argmax_match:.1%}" if r.argmax_match is not None else "n/a"
        lines.append(f"| {r.name} | {_format_float(r.kl_div)} | {_format_float(r.perplexity, 2)} "
                     f"| {am} | {status} |")
    return "\n".join(lines)


def kl_divergence(ref_logits: torch.Tensor, tgt_logits: torch.Tensor) -> float:
    """KL(P_ref || P_tgt) with P = softmax(logits) over the last dimension, averaged over the
    leading rows (quality_metrics.py:70-78)."""
    ref_lp = F.log_softmax(ref_logits.float(), dim=-1)
    tgt_lp = F.log_softmax(tgt_logits.float(), dim=-1)
    return float((ref_lp.exp() * (ref_lp - tgt_lp)).sum(dim=-1).mean())


def perplexity_from_logits(logits: torch.Tensor, input_ids: torch.Tensor) -> float:
    """exp(mean next-token NLL) of logits [seq, vocab] (or [1, seq, vocab]) against input_ids
    shifted by one (quality_metrics.py:81-93)."""
    if logits.dim() == 3:
        logits = logits.squeeze(0)
    ids = input_ids.reshape(-1).to(logits.device)
    lp = F.log_softmax(logits[:-1].float(), dim=-1)
    nll = -lp.gather(dim=-1, index=ids[1:].unsqueeze(-1)).squeeze(-1)
    return float(torch.exp(nll.mean()))


def decoder_last_logits(decoder, input_ids: Sequence[int]) -> torch.Tensor:
    """fp32 logits [vocab] of the last prompt position: every earlier token through decode_step,
    the last through decode_step_with_logits (quality_metrics.py:187-213)."""
    ids = [int(t) for t in input_ids]
    if not ids:
        raise ValueError("empty prompt")
    decoder.reset()
    for t in ids[:-1]:
        decoder.decode_step(t)
    _, logits = decoder.decode_step_with_logits(ids[-1])
    return logits.float().cpu()


def evaluate(name: str, decoder, prompt_ids: Sequence[Sequence[int]],
             ref_logits: Sequence[torch.Tensor]) -> QualityResult:
    """Mean KL(P_ref || P_decoder) and argmax agreement over prompts (quality_metrics.py:214-233).
    """
    if len(prompt_ids) != len(ref_logits) or not prompt_ids:
        raise ValueError("one reference logits row per prompt is required")
    total_kl, matches = 0.0, 0
    for ids, ref in zip(prompt_ids, ref_logits):
        got = decoder_last_logits(decoder, ids)
        ref = ref.reshape(-1).float().cpu()
        total_kl += kl_divergence(ref, got)
        matches += int(int(ref.argmax()) == int(got.argmax()))
    n = len(prompt_ids)
    return QualityResult(name, True, total_kl / n, None, matches / n)


def _hf_reference(model_dir: str, prompts: List[str]):
    """HuggingFace reference logits and perplexity (quality_metrics.py:99-144), local files only.
    """
    from transformers import AutoModelForCausalLM, AutoTokenizer
    tok = AutoTokenizer.from_pretrained(model_dir, local_files_only=True)
    model = AutoModelForCausalLM.from_pretrained(model_dir, torch_dtype=torch.bfloat16,
                                                 local_files_only=True).to("cuda").eval()
    ids, logits, ppl = [], [], 0.0
    for p in prompts:
        x = tok(p, return_tensors="pt").input_ids.to("cuda")
        with torch.no_grad():
            out = model(x, use_cache=False)
        ids.append(x[0].tolist())
        logits.append(out.logits[0, -1].float().cpu())
        ppl += perplexity_from_logits(out.logits, x)
    del model
    torch.cuda.empty_cache()
    return ids, logits, QualityResult("HuggingFace", True, 0.0, ppl / len(prompts), 1.0)


def main(argv: Optional[List[str]] = None) -> int:
    """python -m megaqwen_amd.quality --model /path/to/Qwen3-0.6B (a local checkpoint)."""
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--model", required=True, help="local checkpoint directory")
    ap.add_argument("--max-seq-len", type=int, default=512)
    args = ap.parse_args(argv)
    from .generators import MegakernelGenerator
    results = []
    try:
        ids, ref, hf = _hf_reference(args.model, TEST_PROMPTS)
        results.append(hf)
        gen = MegakernelGenerator(args.model, max_seq_len=args.max_seq_len)
        results.append(evaluate("Megakernel (MI355X)", gen.decoder, ids, ref))
    except Exception as exc:  # reported in the table, as the reference does
        results.append(QualityResult("Megakernel (MI355X)", False, None, None, None, str(exc)))
    print(format_markdown_table(results))
    return 0 if all(r.supported for r in results) else 1


if __name__ == "__main__":
    sys.exit(main())
