"""Which requests a resident epoch may serve.

Mirrors src/vllm_ascend_resident_epoch/eligibility.py:4-47: the epoch runs
plain greedy decoding to EOS or max_tokens, so anything that changes the
sampled token, adds a stop condition or needs per-token host work is
rejected with the reference's reason string (the first that applies).
"""
from __future__ import annotations

from typing import Any


def _request_feature_reason(request: Any) -> str | None:
    checks = (
        (request.pooling_params is not None, "pooling-request"),
        (bool(request.mm_features), "multimodal-input"),
        (request.lora_request is not None, "lora"),
        (request.prompt_embeds is not None, "prompt-embeds"),
        (bool(request.use_structured_output), "structured-output"),
    )
    return next((reason for hit, reason in checks if hit), None)


def _sampling_reason(p: Any) -> str | None:
    checks = (
        (p.temperature != 0.0, "non-greedy-temperature"),
        (p.top_p != 1.0 or p.top_k != 0 or p.min_p != 0.0, "unsupported-sampling-filter"),
        (p.presence_penalty != 0.0 or p.frequency_penalty != 0.0 or p.repetition_penalty != 1.0, "sampling-penalty"),
        (p.min_tokens != 0, "min-tokens"),
        (bool(p.ignore_eos), "ignore-eos"),
        (p.eos_token_id is None, "missing-eos"),
        (bool(p.stop) or bool(p.stop_token_ids), "extra-stop-condition"),
        (p.logprobs is not None or p.prompt_logprobs is not None, "logprobs"),
        (bool(p.logit_bias) or bool(p.allowed_token_ids), "logit-processor"),
        (bool(p.bad_words), "bad-words"),
        (p.repetition_detection is not None, "repetition-detection"),
        (bool(p.extra_args), "extra-sampling-args"),
    )
    return next((reason for hit, reason in checks if hit), None)


def request_rejection_reason(request: Any) -> str | None:
    """None when the request may run in a resident epoch, else the reason."""
    reason = _request_feature_reason(request)
    if reason is not None:
        return reason
    params = request.sampling_params
    if params is None:
        return "missing-sampling-params"
    return _sampling_reason(params)
