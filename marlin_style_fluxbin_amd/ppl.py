"""Teacher-forced batch-1 perplexity through the packed W3 M=1 route.

Protocol of the reference's packed-M=1 PPL runner
(``scripts/run_qwen3_8b_w3_packed_m1_ppl.py``; scoring :230-329, route smoke
:204-227, comparison :338-347, arms and model loading :32 and
``scripts/run_qwen3_8b_w3_full_m1_trial.py:344-375``), kept as the contract:

* three arms on one token stream: ``original_bf16`` (the checkpoint as is),
  ``decoded_w3_bf16`` (every Linear weight replaced by the artifact's restored
  bf16 weight) and ``packed_w3_inline`` (every Linear a ``PackedW3Linear`` from
  the hash-bound artifact, bound for prepared decode);
* every transition of every block is scored by its own one-token forward call
  on a cache that starts empty at each block (teacher forcing, ``use_cache``,
  ``logits_to_keep=1``); its NLL is ``logsumexp(z) - z[label]`` over the fp32
  logits; a block's NLLs are summed in float64, blocks with ``math.fsum``; the
  perplexity is ``exp(total / transitions)`` when that is finite, and an arm stops
  at the first block whose sum is not finite;
* before scoring, the packed arm's route smoke: one call must take ``packed_m1``
  exactly once on every packed Linear;
* the result keys of each arm, the three comparisons and the summary's status
  words.

Not carried: the reference's A100 / Python / library version gates.  In place of
its CUDA extension-cache manifests every arm's provenance holds the kernel
library's build contract key and library digest (``w3_lut_extension_build``: this
build loads one prebuilt HIP library, which fails loudly when absent), so a
resumed run refuses arms scored by other kernels.  Tokens come from a safetensors file holding one
``tokens`` tensor, checked against expected hashes when they are given, and cut
into blocks of ``sequence_length``.

Organisation here: ``_TransitionScorer`` owns the per-block loop for one model;
``score_m1_ppl`` aggregates blocks into the arm record; ``run_ppl`` runs the arms
one model at a time, writing each arm's record atomically (so ``resume`` skips
finished arms) and then the summary.
"""
from __future__ import annotations

import argparse
import datetime as dt
import hashlib
import json
import math
import struct
import time
from contextlib import ExitStack
from pathlib import Path
from typing import Callable, Iterable, Sequence

import torch

ARMS = ("original_bf16", "decoded_w3_bf16", "packed_w3_inline")
PACKED_ARM = "packed_w3_inline"


# ----------------------------------------------------------------- token stream
def sha256_token_sequences(sequences: Iterable[Sequence[int]]) -> str:
    """Hash of token sequences with explicit framing: per sequence its length as a
    big-endian uint64, then each token as a big-endian int64 (the reference's
    ``evaluation.py:37-45`` record format, so hashes recorded there compare)."""
    digest = hashlib.sha256()
    for sequence in sequences:
        values = [int(t) for t in sequence]
        digest.update(struct.pack(">Q", len(values)))
        digest.update(struct.pack(f">{len(values)}q", *values))
    return digest.hexdigest()


def token_blocks(tokens: Sequence[int], sequence_length: int, *, used_token_count: int | None = None) -> list[list[int]]:
    """Consecutive blocks of ``sequence_length`` tokens over the first
    ``used_token_count`` tokens (default: every whole block of the stream)."""
    if sequence_length < 2:
        raise ValueError("a PPL block needs at least two tokens")
    if used_token_count is None:
        used_token_count = len(tokens) // sequence_length * sequence_length
    if not 0 < used_token_count <= len(tokens) or used_token_count % sequence_length:
        raise ValueError(f"used_token_count {used_token_count} must be a positive multiple of "
                         f"{sequence_length} within the {len(tokens)} tokens")
    stream = [int(t) for t in tokens[:used_token_count]]
    return [stream[i:i + sequence_length] for i in range(0, used_token_count, sequence_length)]


def load_token_artifact(path: Path, *, expected_file_sha256: str | None = None,
                        expected_tokens_sha256: str | None = None) -> list[int]:
    """The ``tokens`` tensor of a safetensors file, after its hash gates."""
    from safetensors import safe_open

    from .w3_lut_artifacts import sha256_file

    path = Path(path)
    if expected_file_sha256 is not None and sha256_file(path) != expected_file_sha256:
        raise ValueError("token artifact hash drifted")
    with safe_open(str(path), framework="pt", device="cpu") as source:
        if set(source.keys()) != {"tokens"}:
            raise ValueError("token artifact inventory drifted: expected exactly one 'tokens' tensor")
        tensor = source.get_tensor("tokens")
    if tensor.dtype not in (torch.int32, torch.int64) or tensor.ndim != 1:
        raise ValueError(f"tokens must be a 1-D int32/int64 tensor, got {tensor.dtype} {tuple(tensor.shape)}")
    tokens = tensor.tolist()
    if expected_tokens_sha256 is not None and sha256_token_sequences([tokens]) != expected_tokens_sha256:
        raise ValueError("token stream hash drifted")
    return tokens


# ----------------------------------------------------------------- scoring
def finite_perplexity(mean_nll: float | None) -> float | None:
    """``exp(mean_nll)`` when both are finite, else None."""
    if mean_nll is None or not math.isfinite(mean_nll) or mean_nll > 709.0:
        return None
    value = math.exp(mean_nll)
    return value if math.isfinite(value) else None


def _cache_length(cache) -> int:
    length = cache.get_seq_length()
    return int(length.item()) if isinstance(length, torch.Tensor) else int(length)


class _TransitionScorer:
    """One-token cached forward calls over a block; fp32 NLL of each transition."""

    def __init__(self, model, device: torch.device):
        self.model, self.device = model, device
        self.logits_dtype = None

    def step(self, token: torch.Tensor, cache):
        output = self.model(input_ids=token.view(1, 1), past_key_values=cache, use_cache=True, logits_to_keep=1)
        self.logits_dtype = str(output.logits.dtype)
        return output.logits[0, -1].float(), output.past_key_values

    def block(self, block: Sequence[int]) -> torch.Tensor:
        if len(block) < 2:
            raise ValueError("PPL block must contain at least two tokens")
        ids = torch.tensor(block, dtype=torch.long, device=self.device)
        nll = torch.empty(len(block) - 1, dtype=torch.float32, device=self.device)
        cache = None
        for position in range(len(block) - 1):
            logits, cache = self.step(ids[position], cache)
            nll[position] = torch.logsumexp(logits, dim=0) - logits[ids[position + 1]]
        if _cache_length(cache) != len(block) - 1:
            raise RuntimeError("KV cache length drifted during M=1 PPL")
        return nll


def _reset_routes(modules: dict) -> None:
    for module in modules.values():
        module.reset_route_counts()


@torch.inference_mode()
def packed_route_smoke(model, token: int, device: torch.device, *, expected_linears: int | None = None) -> dict | None:
    """One audited one-token call: every packed Linear must count exactly one
    ``packed_m1`` call and no fallback (None when the model has no packed Linear)."""
    from .full_model_trial import packed_modules

    modules = packed_modules(model)
    if not modules:
        return None
    _reset_routes(modules)
    for module in modules.values():
        module._decode_audit = True
    try:
        model(input_ids=torch.tensor([[token]], dtype=torch.long, device=device), use_cache=True, logits_to_keep=1)
    finally:
        for module in modules.values():
            module._decode_audit = False
    expected = expected_linears if expected_linears is not None else len(modules)
    clean = all(module.route_counts.get("packed_m1") == 1 and
                sum(module.route_counts.values()) == 1 for module in modules.values())
    if len(modules) != expected or not clean:
        raise RuntimeError("packed M=1 route smoke failed")
    return {"passed": True, "linear_count": len(modules), "calls_per_linear": 1}


def _tensor_sha256(values: torch.Tensor) -> str:
    return hashlib.sha256(values.detach().cpu().numpy().tobytes()).hexdigest()


@torch.inference_mode()
def score_m1_ppl(model, blocks: list[list[int]], *, arm: str, device: torch.device, expected_packed_linears: int,
                 progress: Callable[[int, int], None] | None = None) -> dict:
    """Score every transition of ``blocks`` with one-token cached calls; the arm record."""
    from .full_model_trial import packed_modules
    from .static_decode import prepared_linears

    if model.training:
        raise ValueError("PPL model must be in eval mode")
    if not blocks:
        raise ValueError("no PPL blocks")
    gpu = device.type == "cuda"
    if gpu:
        torch.cuda.reset_peak_memory_stats(device)
        torch.cuda.synchronize(device)
    started = time.monotonic()
    scorer = _TransitionScorer(model, device)
    sums, hashes, nonfinite = [], [], []
    transitions = 0
    with ExitStack() as stack:
        if expected_packed_linears:
            modules = stack.enter_context(prepared_linears(model, torch.bfloat16))
            if len(modules) != expected_packed_linears:
                raise RuntimeError(f"packed Linear count drifted for {arm}: {len(modules)} != {expected_packed_linears}")
        elif packed_modules(model):
            raise RuntimeError(f"arm {arm} expects no packed Linear")
        smoke = packed_route_smoke(model, blocks[0][0], device, expected_linears=expected_packed_linears or None)
        for index, block in enumerate(blocks):
            nll = scorer.block(block)
            total = float(nll.double().sum())
            if not math.isfinite(total):
                nonfinite.append(index)
                break
            sums.append(total)
            hashes.append(_tensor_sha256(nll))
            transitions += len(block) - 1
            if progress is not None:
                progress(index + 1, len(blocks))
    if gpu:
        torch.cuda.synchronize(device)
    total_nll = math.fsum(sums) if not nonfinite else None
    mean_nll = total_nll / transitions if total_nll is not None else None
    perplexity = finite_perplexity(mean_nll)
    valid = perplexity is not None and not nonfinite
    return {
        "arm": arm,
        "status": "completed" if valid else "invalid",
        "execution": "teacher_forced_cached_decode_m1",
        "tokens_per_model_call": 1,
        "block_count": len(sums),
        "scored_transition_count": transitions,
        "total_nll": total_nll,
        "mean_nll": mean_nll,
        "perplexity": perplexity,
        "metrics_valid": valid,
        "nonfinite_block_indices": nonfinite,
        "block_nll_sha256": hashes,
        "logits_dtype": scorer.logits_dtype,
        "nll_logits_dtype": "torch.float32",
        "elapsed_seconds": time.monotonic() - started,
        "peak_allocated_bytes": torch.cuda.max_memory_allocated(device) if gpu else None,
        "packed_route_smoke": smoke,
        "packed_linear_count": len(packed_modules(model)),
        "dense_fallback_permitted_during_scoring": False,
    }


def comparison(candidate: dict, baseline: dict) -> dict:
    """PPL and mean-NLL differences of two arm records."""
    cp, bp = candidate["perplexity"], baseline["perplexity"]
    return {
        "candidate": candidate["arm"],
        "baseline": baseline["arm"],
        "ppl_delta": cp - bp,
        "ppl_relative_percent": (cp / bp - 1.0) * 100.0,
        "mean_nll_delta": candidate["mean_nll"] - baseline["mean_nll"],
    }


# ----------------------------------------------------------------- arms
@torch.inference_mode()
def prepare_arm(model, arm: str, *, artifact_root: Path, expected_manifest_sha256: str) -> dict | None:
    """Turn a freshly loaded bf16 model into ``arm`` in place; the coverage record
    of the packed arm (None for the dense arms)."""
    from .gptq_deployment import FIELDS, restore_planar_w3
    from .qwen3 import QWEN3_LINEAR_MODULES
    from .w3_lut_artifacts import load_w3_lut_layer, replace_w3_model_linears

    if arm not in ARMS:
        raise ValueError(f"unknown PPL arm {arm}")
    if arm == "decoded_w3_bf16":
        for index, block in enumerate(model.model.layers):
            tensors, _ = load_w3_lut_layer(artifact_root, index, expected_manifest_sha256=expected_manifest_sha256)
            for name in QWEN3_LINEAR_MODULES:
                linear = block.get_submodule(name)
                layout = {f: tensors[f"{name}.{f}"].to(linear.weight.device) for f in FIELDS}
                linear.weight.copy_(restore_planar_w3(layout, dtype=linear.weight.dtype))
        return None
    if arm == PACKED_ARM:
        coverage = replace_w3_model_linears(model, artifact_root, expected_manifest_sha256=expected_manifest_sha256,
                                            allow_prefill_fallback=True, route="structural")
        expected = len(QWEN3_LINEAR_MODULES) * len(model.model.layers)
        if coverage["linear_count"] != expected:
            raise RuntimeError("incomplete packed W3 coverage")
        return coverage
    return None


def _write_json(path: Path, value: dict) -> None:
    tmp = path.with_name(path.name + ".tmp")
    tmp.write_text(json.dumps(value, indent=1, sort_keys=True) + "\n", encoding="utf-8")
    tmp.replace(path)


def run_ppl(load_model: Callable[[], torch.nn.Module], blocks: list[list[int]], *, artifact_root: Path,
            expected_manifest_sha256: str, output_dir: Path, device: torch.device, arms: Sequence[str] = ARMS,
            resume: bool = False, seed: int = 0, provenance: dict | None = None, fused_modules: bool = True) -> dict:
    """Score ``arms`` one model at a time (``load_model()`` returns a fresh eval
    bf16 model on ``device``) and write ``arms/<arm>.json`` and ``summary.json``."""
    from .fused_modules import fused_qwen3_modules

    output_dir = Path(output_dir)
    from .w3_lut_deployment import w3_lut_extension_build

    _, build = w3_lut_extension_build(256)  # one library: the same contract for every row tile
    provenance = dict(provenance or {}, blocks_sha256=sha256_token_sequences(blocks),
                      w3_layout_manifest_sha256=expected_manifest_sha256,
                      w3_kernel_build_cache_key=build["cache_key"], w3_kernel_library_sha256=build["library_sha256"])
    if resume:
        if not (output_dir / "arms").is_dir():
            raise FileNotFoundError(output_dir / "arms")
    else:
        if output_dir.exists():
            raise FileExistsError(output_dir)
        (output_dir / "arms").mkdir(parents=True)
    unknown = set(arms) - set(ARMS)
    if unknown:
        raise ValueError(f"unknown PPL arms {sorted(unknown)}")
    metrics, coverage = {}, {}
    with ExitStack() as stack:
        if fused_modules:
            stack.enter_context(fused_qwen3_modules(rms_norm=True, rope=True))
        for arm in arms:
            path = output_dir / "arms" / f"{arm}.json"
            if resume and path.is_file():
                record = json.loads(path.read_text(encoding="utf-8"))
                if record.get("provenance") != provenance or not record.get("metrics", {}).get("metrics_valid"):
                    raise ValueError(f"invalid resumable arm: {arm}")
                metrics[arm] = record["metrics"]
                continue
            torch.manual_seed(seed)
            model = load_model()
            model.config.use_cache = True
            coverage[arm] = prepare_arm(model, arm, artifact_root=artifact_root,
                                        expected_manifest_sha256=expected_manifest_sha256)
            expected = coverage[arm]["linear_count"] if arm == PACKED_ARM else 0
            metrics[arm] = score_m1_ppl(model, blocks, arm=arm, device=device, expected_packed_linears=expected)
            _write_json(path, {"schema_version": 1, "provenance": provenance, "coverage": coverage[arm],
                               "metrics": metrics[arm]})
            del model
            if device.type == "cuda":
                torch.cuda.empty_cache()
    validity = {arm: bool(metrics[arm]["metrics_valid"] and metrics[arm]["block_count"] == len(blocks)
                          and (arm != PACKED_ARM or (metrics[arm]["packed_route_smoke"] or {}).get("passed")))
                for arm in arms}
    pairs = (("decoded_w3_vs_original_bf16", "decoded_w3_bf16", "original_bf16"),
             ("packed_w3_vs_decoded_w3", PACKED_ARM, "decoded_w3_bf16"),
             ("packed_w3_vs_original_bf16", PACKED_ARM, "original_bf16"))
    comparisons = {name: comparison(metrics[a], metrics[b]) for name, a, b in pairs
                   if a in metrics and b in metrics and validity.get(a) and validity.get(b)}
    summary = {
        "schema_version": 1,
        "status": "completed_pending_effect_size_review" if all(validity.values()) else "completed_invalid_metrics",
        "created_at_utc": dt.datetime.now(dt.timezone.utc).isoformat(),
        "provenance": provenance,
        "arms": metrics,
        "validity_gates": validity,
        "comparisons": comparisons,
        "quality_effect_threshold": None,
        "decision": "manual_effect_size_review",
        "performance_claim": None,
    }
    _write_json(output_dir / "summary.json", summary)
    return summary


def main(argv=None) -> dict:
    """``python -m marlin_style_fluxbin_amd.ppl --snapshot-root DIR --token-artifact FILE
    --w3-layout-root DIR --w3-layout-manifest-sha256 HEX --output-dir DIR``."""
    from .w3_lut_artifacts import sha256_file

    parser = argparse.ArgumentParser(description="teacher-forced M=1 PPL through the packed W3 route")
    parser.add_argument("--snapshot-root", type=Path, required=True, help="local HF Qwen3 checkpoint directory")
    parser.add_argument("--token-artifact", type=Path, required=True)
    parser.add_argument("--token-artifact-sha256")
    parser.add_argument("--tokens-sha256")
    parser.add_argument("--sequence-length", type=int, default=2048)
    parser.add_argument("--used-token-count", type=int)
    parser.add_argument("--max-blocks", type=int, help="score only the first N blocks (a bounded sample)")
    parser.add_argument("--w3-layout-root", type=Path, required=True)
    parser.add_argument("--w3-layout-manifest-sha256", required=True)
    parser.add_argument("--output-dir", type=Path, required=True)
    parser.add_argument("--arms", nargs="+", default=list(ARMS), choices=list(ARMS))
    parser.add_argument("--device", default="cuda:0")
    parser.add_argument("--seed", type=int, default=20260917)
    parser.add_argument("--resume", action="store_true")
    args = parser.parse_args(argv)

    if sha256_file(args.w3_layout_root / "manifest.json") != args.w3_layout_manifest_sha256:
        raise ValueError("W3 layout manifest drifted")
    tokens = load_token_artifact(args.token_artifact, expected_file_sha256=args.token_artifact_sha256,
                                 expected_tokens_sha256=args.tokens_sha256)
    blocks = token_blocks(tokens, args.sequence_length, used_token_count=args.used_token_count)
    if args.max_blocks is not None:
        blocks = blocks[:args.max_blocks]
    device = torch.device(args.device)
    if device.type == "cuda":
        torch.cuda.set_device(device)
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False

    def load_model():
        from transformers import AutoModelForCausalLM

        return AutoModelForCausalLM.from_pretrained(args.snapshot_root, local_files_only=True, dtype=torch.bfloat16,
                                                    attn_implementation="sdpa").to(device).eval()

    provenance = {"token_artifact_sha256": sha256_file(args.token_artifact),
                  "snapshot_config_sha256": sha256_file(args.snapshot_root / "config.json")}
    summary = run_ppl(load_model, blocks, artifact_root=args.w3_layout_root,
                      expected_manifest_sha256=args.w3_layout_manifest_sha256, output_dir=args.output_dir,
                      device=device, arms=args.arms, resume=args.resume, seed=args.seed, provenance=provenance)
    for arm, record in summary["arms"].items():
        print(f"{arm} ppl={record['perplexity']} transitions={record['scored_transition_count']}", flush=True)
    print(summary["status"], flush=True)
    return summary


if __name__ == "__main__":
    main()
