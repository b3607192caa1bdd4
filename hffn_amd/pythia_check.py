"""End-to-end parity of the HFFN arm of a Pythia model against its dense arm, on synthetic prompts
(the criterion of ``runtime/common/pythia/hffn_pythia/parity_model.py:1-126``).

Three models from the same checkpoint and export, on the same device: the dense arm and the HFFN arm in float32, and
the dense arm in float64 as the arbiter. Compared tokens: the argmax at every prefill position, then at every step of
a cached greedy decode in which the three models are fed the arbiter's token, so that they always see the same
context. A token passes if it equals the dense float32 token, or the float64 token, or if its float64 margin (float64
token's logit minus the chosen token's logit) is at most the larger of one float32 step and the dense float32
control's own error at that position (``parity_model.py:10-17,104-118``): on a near tie that the float32 control
cannot resolve either, a different argmax is not a fault of the HFFN arm. The negative control scales
``attention.dense.weight`` of layer 3 of an HFFN arm by 1.5 and must report unexplained tokens.

    python -m hffn_amd.pythia_check --workdir /tmp/pythia410m [--batch 8 --length 512 --steps 128]
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import torch

FAULT_LAYER, FAULT_SCALE = 3, 1.5


@torch.inference_mode()
def all_logits(models: list, prompt: torch.Tensor, steps: int) -> list[torch.Tensor]:
    """Per model, its logits [B, T + steps, vocabulary]; ``models[-1]`` drives the decode (``parity_model.py:36-46``)."""
    outputs = [model(input_ids=prompt, use_cache=True) for model in models]
    logits = [[output.logits] for output in outputs]
    for _ in range(steps):
        fed = outputs[-1].logits[:, -1:].argmax(-1)
        outputs = [model(input_ids=fed, past_key_values=output.past_key_values, use_cache=True) for model, output in zip(models, outputs)]
        for kept, output in zip(logits, outputs):
            kept.append(output.logits)
    return [torch.cat(kept, dim=1) for kept in logits]


def float32_step(value: torch.Tensor) -> torch.Tensor:
    """Distance from each |value| to the next float32 (``parity_model.py:49-52``)."""
    magnitude = value.abs().float()
    return (torch.nextafter(magnitude, torch.full_like(magnitude, float("inf"))) - magnitude).double()


@torch.inference_mode()
def inject_fault(model, layer: int = FAULT_LAYER) -> None:
    """The negative control's predeclared fault: one dense weight of the HFFN arm only, scaled."""
    model.gpt_neox.layers[layer].attention.dense.weight.mul_(FAULT_SCALE)


def check_arm(dense, hffn, arbiter, prompts: list[torch.Tensor], steps: int, log=print) -> dict:
    """The check of one HFFN arm against the dense float32 control and the float64 arbiter (``parity_model.py:95-126``);
    returns the counts (``unexplained`` must be 0)."""
    totals = {"tokens": 0, "differs": 0, "moved": 0, "one_step": 0, "by_band": 0, "unexplained": 0, "dense_vs_float64": 0,
              "largest_band": 0.0, "prefill_max_dlogit": 0.0}
    for prompt in prompts:
        dense_logits, hffn_logits, arbiter_logits = all_logits([dense, hffn, arbiter], prompt, steps)
        dense_tokens, hffn_tokens, arbiter_tokens = dense_logits.argmax(-1), hffn_logits.argmax(-1), arbiter_logits.argmax(-1)
        differs = hffn_tokens != dense_tokens
        moved = differs & (hffn_tokens != arbiter_tokens)
        best = arbiter_logits.gather(-1, arbiter_tokens.unsqueeze(-1)).squeeze(-1)
        chosen = arbiter_logits.gather(-1, hffn_tokens.unsqueeze(-1)).squeeze(-1)
        margin, step = best - chosen, float32_step(best)
        dense64 = dense_logits.double()
        control_error = ((dense64.gather(-1, arbiter_tokens.unsqueeze(-1)).squeeze(-1) - best).abs()
                         + (dense64.gather(-1, hffn_tokens.unsqueeze(-1)).squeeze(-1) - chosen).abs())
        band = torch.maximum(step, control_error)
        wrong = moved & (margin > band)
        one_step = moved & (margin <= step)
        by_band = moved & (margin > step) & ~wrong
        length = prompt.shape[1]
        gap = float((hffn_logits[:, :length] - dense_logits[:, :length]).abs().max())
        counts = {"tokens": hffn_tokens.numel(), "differs": int(differs.sum()), "moved": int(moved.sum()),
                  "one_step": int(one_step.sum()), "by_band": int(by_band.sum()), "unexplained": int(wrong.sum()),
                  "dense_vs_float64": int((dense_tokens != arbiter_tokens).sum())}
        for key, value in counts.items():
            totals[key] += value
        totals["largest_band"] = max(totals["largest_band"], float(band.max()))
        totals["prefill_max_dlogit"] = max(totals["prefill_max_dlogit"], gap)
        log(f"B={prompt.shape[0]} T={length}: {counts['tokens']} tokens, hffn != dense32 {counts['differs']} (of which "
            f"!= float64: {counts['moved']}, within one float32 step: {counts['one_step']}, within the control band: "
            f"{counts['by_band']}, unexplained: {counts['unexplained']}), dense32 != float64 {counts['dense_vs_float64']}; "
            f"prefill max|dlogit| {gap:.2e}; max band {float(band.max()):.2e}")
    return totals


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
        start = time.time()
        pythia.write_random_pythia(model_dir, export_dir, seed=args.seed, num_hidden_layers=args.layers)
        print(f"wrote random-init Pythia-410M-shape model ({args.layers} layers) in {time.time() - start:.1f} s", flush=True)
    device = torch.device("cuda", 0)
    dense = pythia.load_pythia(model_dir, export_dir, "dense", device)
    hffn = pythia.load_pythia(model_dir, export_dir, "hffn", device)
    arbiter = pythia.load_pythia(model_dir, export_dir, "dense", device).double()
    print(f"loaded the dense, HFFN and float64 arms; prompts {args.batch} x {args.length}, {args.steps} decode steps",
          flush=True)
    vocab = dense.config.vocab_size
    prompts = [pythia.synthetic_prompts(args.batch, args.length, vocab).to(device)]
    result = check_arm(dense, hffn, arbiter, prompts, args.steps, log=lambda s: print(s, flush=True))
    result["calls"] = {f"{up}/{down}": count for (up, down), count in hffn.hffn_runtime.calls.items()}
    print(json.dumps(result), flush=True)
    code = 0 if result["unexplained"] == 0 else 1
    if args.negative_control:
        faulty = pythia.load_pythia(model_dir, export_dir, "hffn", device)
        inject_fault(faulty)
        found = check_arm(dense, faulty, arbiter, prompts, args.steps, log=lambda s: print(s, flush=True))["unexplained"]
        print(f"negative control (layer {FAULT_LAYER} attention.dense.weight x {FAULT_SCALE}): {found} unexplained tokens -> "
              f"{'DETECTED' if found else 'NOT DETECTED'}", flush=True)
        code = code or (0 if found else 1)
    return code


if __name__ == "__main__":
    sys.exit(main())
