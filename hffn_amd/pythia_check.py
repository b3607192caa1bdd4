"""Greedy-token parity of the HFFN arm of a Pythia model on synthetic prompts.

The criterion is the reference's (``runtime/common/pythia/hffn_pythia/parity_model.py:1-20,104-118``); its code here
is this package's own. Three models share a checkpoint and an export: the dense arm and the HFFN arm in float32, and
the dense arm in float64 (the arbiter). They run in lockstep over a prompt and then a cached greedy decode fed with the
arbiter's tokens, so that all three always see the same context. At every position each model's argmax is a token;
the HFFN token is classified as

* ``dense``   - equal to the dense float32 token;
* ``float64`` - otherwise equal to the arbiter's token;
* ``ulp``     - otherwise within one float32 step of the arbiter's best logit, measured on the arbiter's logits;
* ``control`` - otherwise within the dense float32 control's own error at that position (its distance to the
  arbiter on the arbiter's token plus on the HFFN token);
* ``unexplained`` - anything else, which fails the check.

The negative control multiplies ``attention.dense.weight`` of one layer of an HFFN arm by 1.5; the check must then
report unexplained tokens.

    python -m hffn_amd.pythia_check --workdir /tmp/pythia410m [--batch 8 --length 512 --steps 128] [--negative-control]
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import torch

FAULT_LAYER, FAULT_SCALE = 3, 1.5
CLASSES = ("dense", "float64", "ulp", "control", "unexplained")


class Lockstep:
    """Models decoded together: the prompt once, then one cached step at a time, every model fed the token the last
    model (the arbiter) picks. Keeps each model's logits of every position."""

    def __init__(self, models: list) -> None:
        self.models = models
        self.caches = [None] * len(models)
        self.logits: list[list[torch.Tensor]] = [[] for _ in models]

    def _feed(self, tokens: torch.Tensor) -> None:
        for k, model in enumerate(self.models):
            out = model(input_ids=tokens, past_key_values=self.caches[k], use_cache=True)
            self.caches[k] = out.past_key_values
            self.logits[k].append(out.logits)

    @torch.inference_mode()
    def run(self, prompt: torch.Tensor, steps: int) -> list[torch.Tensor]:
        self._feed(prompt)
        for _ in range(steps):
            self._feed(self.logits[-1][-1][:, -1:].argmax(-1))
        return [torch.cat(kept, dim=1) for kept in self.logits]


def float32_spacing(value: torch.Tensor) -> torch.Tensor:
    """Gap between |value| (rounded to float32) and the next float32 up, in float64: 2^(e - 24) for |value| in
    [2^(e-1), 2^e), and the subnormal step 2^-149 below the normal range (zero included)."""
    magnitude = value.abs().float()
    _, exponent = torch.frexp(magnitude)
    spacing = torch.ldexp(torch.ones_like(magnitude, dtype=torch.float64), (exponent - 24).to(torch.int32))
    return torch.where(magnitude < 2.0 ** -126, torch.full_like(spacing, 2.0 ** -149), spacing)


def classify(dense_logits: torch.Tensor, hffn_logits: torch.Tensor, arbiter_logits: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per position, the index in ``CLASSES`` of the HFFN token, and the tolerance band used (float64)."""
    pick = lambda logits, tokens: logits.gather(-1, tokens.unsqueeze(-1)).squeeze(-1).double()  # noqa: E731
    dense_token, hffn_token, arbiter_token = (l.argmax(-1) for l in (dense_logits, hffn_logits, arbiter_logits))
    best, chosen = pick(arbiter_logits, arbiter_token), pick(arbiter_logits, hffn_token)
    shortfall = best - chosen
    ulp = float32_spacing(best)
    control = (pick(dense_logits, arbiter_token) - best).abs() + (pick(dense_logits, hffn_token) - chosen).abs()
    band = torch.maximum(ulp, control)
    code = torch.full_like(hffn_token, CLASSES.index("unexplained"))
    for name, holds in reversed((("dense", hffn_token == dense_token), ("float64", hffn_token == arbiter_token),
                                 ("ulp", shortfall <= ulp), ("control", shortfall <= band))):
        code = torch.where(holds, torch.full_like(code, CLASSES.index(name)), code)
    return code, band


def check_arm(dense, hffn, arbiter, prompts: list[torch.Tensor], steps: int, log=print) -> dict:
    """The token check of one HFFN arm against the dense float32 control and the float64 arbiter over ``prompts``
    ([B, T] token tensors on the models' device), ``steps`` decode steps each. Returns the counts per class (the check
    passes when ``unexplained`` is 0), how often the dense float32 arm itself disagreed with the arbiter, the widest
    band used and the largest prefill logit gap between the HFFN and the dense arm."""
    report = {name: 0 for name in CLASSES}
    report.update(tokens=0, dense_vs_float64=0, largest_band=0.0, prefill_max_dlogit=0.0)
    for prompt in prompts:
        dense_logits, hffn_logits, arbiter_logits = Lockstep([dense, hffn, arbiter]).run(prompt, steps)
        code, band = classify(dense_logits, hffn_logits, arbiter_logits)
        counts = torch.bincount(code.flatten(), minlength=len(CLASSES)).tolist()
        prefill_gap = float((hffn_logits[:, :prompt.shape[1]] - dense_logits[:, :prompt.shape[1]]).abs().max())
        control_misses = int((dense_logits.argmax(-1) != arbiter_logits.argmax(-1)).sum())
        for name, count in zip(CLASSES, counts):
            report[name] += count
        report["tokens"] += code.numel()
        report["dense_vs_float64"] += control_misses
        report["largest_band"] = max(report["largest_band"], float(band.max()))
        report["prefill_max_dlogit"] = max(report["prefill_max_dlogit"], prefill_gap)
        log(f"prompt {tuple(prompt.shape)} + {steps} steps: " + ", ".join(f"{n} {c}" for n, c in zip(CLASSES, counts))
            + f"; dense32 vs float64 argmax {control_misses}; prefill max|dlogit| {prefill_gap:.2e}; "
              f"widest band {float(band.max()):.2e}")
    return report


@torch.inference_mode()
def inject_fault(model, layer: int = FAULT_LAYER) -> None:
    """The negative control's predeclared fault, applied to the HFFN arm only."""
    model.gpt_neox.layers[layer].attention.dense.weight.mul_(FAULT_SCALE)


def main(argv: list[str] | None = None) -> int:
    from . import pythia
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--workdir", type=Path, required=True, help="holds model/ and export/ (written when missing)")
    parser.add_argument("--batch", type=int, default=8)
    parser.add_argument("--length", type=int, default=512)
    parser.add_argument("--steps", type=int, default=128)
    parser.add_argument("--layers", type=int, default=24)
    parser.add_argument("--seed", type=int, default=104)
    parser.add_argument("--negative-control", action="store_true")
    args = parser.parse_args(argv)
    model_dir, export_dir = args.workdir / "model", args.workdir / "export"
    if not (model_dir / "model.safetensors").exists():
        began = time.time()
        pythia.write_random_pythia(model_dir, export_dir, seed=args.seed, num_hidden_layers=args.layers)
        print(f"random-init Pythia-410M-shape model with {args.layers} layers written in {time.time() - began:.1f} s", flush=True)
    device = torch.device("cuda", 0)
    arms = {ffn: pythia.load_pythia(model_dir, export_dir, ffn, device) for ffn in ("dense", "hffn")}
    arbiter = pythia.load_pythia(model_dir, export_dir, "dense", device).double()
    prompts = [pythia.synthetic_prompts(args.batch, args.length, arms["dense"].config.vocab_size).to(device)]
    print(f"three arms loaded; {args.batch} prompts of {args.length} tokens, {args.steps} greedy steps", flush=True)
    say = lambda line: print(line, flush=True)  # noqa: E731
    report = check_arm(arms["dense"], arms["hffn"], arbiter, prompts, args.steps, log=say)
    report["calls"] = {f"{up}/{down}": count for (up, down), count in arms["hffn"].hffn_runtime.calls.items()}
    print(json.dumps(report), flush=True)
    failed = report["unexplained"] != 0
    if args.negative_control:
        faulty = pythia.load_pythia(model_dir, export_dir, "hffn", device)
        inject_fault(faulty)
        caught = check_arm(arms["dense"], faulty, arbiter, prompts, args.steps, log=say)["unexplained"]
        print(f"negative control, layer {FAULT_LAYER} attention.dense.weight scaled by {FAULT_SCALE}: {caught} tokens "
              f"unexplained -> {'caught' if caught else 'MISSED'}", flush=True)
        failed = failed or caught == 0
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
