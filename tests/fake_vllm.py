"""A small in-memory stand-in for vLLM v1's scheduler, request and output
records (vLLM is not installed here), with the behaviour the resident-epoch
scheduler relies on:

* ``schedule`` serves running requests first (each for the tokens it has
  not computed yet), then admits waiting requests while fewer than
  ``max_num_running_reqs`` run, scheduling their whole prompt; every
  scheduled request's ``num_computed_tokens`` advances at the end of
  ``schedule`` (vLLM's ``_update_after_schedule``); each admitted request gets
  one KV block of ``block_size`` tokens from a free list.
* ``update_from_output`` appends the sampled tokens, stopping at EOS or
  ``max_tokens`` (status FINISHED_STOPPED / FINISHED_LENGTH_CAPPED), and
  frees finished requests' blocks and running slots.

Test infrastructure only.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from types import SimpleNamespace

EOS_TOKEN_ID = 151645


class RequestStatus(Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED_STOPPED = "finished_stopped"
    FINISHED_LENGTH_CAPPED = "finished_length_capped"


def greedy_params(max_tokens: int, eos: int = EOS_TOKEN_ID, **overrides) -> SimpleNamespace:
    params = SimpleNamespace(
        temperature=0.0, top_p=1.0, top_k=0, min_p=0.0, presence_penalty=0.0, frequency_penalty=0.0,
        repetition_penalty=1.0, min_tokens=0, ignore_eos=False, eos_token_id=eos, stop=[], stop_token_ids=[],
        logprobs=None, prompt_logprobs=None, logit_bias=None, allowed_token_ids=None, bad_words=[],
        repetition_detection=None, extra_args=None, max_tokens=max_tokens, output_kind="cumulative",
    )
    for k, v in overrides.items():
        setattr(params, k, v)
    return params


@dataclass(eq=False)
class Request:
    request_id: str
    prompt_token_ids: list[int]
    sampling_params: SimpleNamespace
    output_token_ids: list[int] = field(default_factory=list)
    num_computed_tokens: int = 0
    status: RequestStatus = RequestStatus.WAITING
    pooling_params: object = None
    mm_features: list = field(default_factory=list)
    lora_request: object = None
    prompt_embeds: object = None
    use_structured_output: bool = False

    @property
    def num_prompt_tokens(self) -> int:
        return len(self.prompt_token_ids)

    @property
    def num_output_tokens(self) -> int:
        return len(self.output_token_ids)

    @property
    def num_tokens(self) -> int:
        return self.num_prompt_tokens + self.num_output_tokens

    @property
    def all_token_ids(self) -> list[int]:
        return self.prompt_token_ids + self.output_token_ids

    @property
    def max_tokens(self) -> int:
        return self.sampling_params.max_tokens


@dataclass
class SchedulerOutput:
    num_scheduled_tokens: dict[str, int]
    scheduled_spec_decode_tokens: dict = field(default_factory=dict)
    scheduled_encoder_inputs: dict = field(default_factory=dict)
    preempted_req_ids: set = field(default_factory=set)


class _Blocks:
    def __init__(self, ids):
        self._ids = ids

    def get_block_ids(self):
        return (list(self._ids),)


class FakeKVCacheManager:
    def __init__(self, num_blocks: int):
        self.free = list(range(num_blocks))
        self.owned: dict[str, list[int]] = {}

    def allocate(self, request_id: str) -> None:
        if request_id not in self.owned:
            self.owned[request_id] = [self.free.pop(0)]

    def release(self, request_id: str) -> None:
        self.free = sorted(self.free + self.owned.pop(request_id, []))

    def get_blocks(self, request_id: str) -> _Blocks:
        return _Blocks(self.owned.get(request_id, []))


def qwen7b_vllm_config(**hf_overrides) -> SimpleNamespace:
    hf = SimpleNamespace(model_type="qwen2", num_hidden_layers=28, hidden_size=3584, vocab_size=152064)
    for k, v in hf_overrides.items():
        setattr(hf, k, v)
    return SimpleNamespace(
        speculative_config=None,
        parallel_config=SimpleNamespace(tensor_parallel_size=1, pipeline_parallel_size=1),
        model_config=SimpleNamespace(hf_config=hf),
    )


class FakeScheduler:
    def __init__(self, max_num_seqs: int = 4, max_num_batched_tokens: int = 128, block_size: int = 128,
                 num_blocks: int = 16, vllm_config=None, async_scheduling: bool = False) -> None:
        self.vllm_config = vllm_config or qwen7b_vllm_config()
        self.scheduler_config = SimpleNamespace(async_scheduling=async_scheduling)
        self.max_num_running_reqs = max_num_seqs
        self.max_num_batched_tokens = max_num_batched_tokens
        self.block_size = block_size
        self.num_lookahead_tokens = 0
        self.connector = None
        self.ec_connector = None
        self.kv_cache_manager = FakeKVCacheManager(num_blocks)
        self.requests: dict[str, Request] = {}
        self.running: list[Request] = []
        self.waiting: list[Request] = []
        self.skipped_waiting: list[Request] = []

    def add_request(self, request: Request) -> None:
        self.requests[request.request_id] = request
        self.waiting.append(request)

    def schedule(self) -> SchedulerOutput:
        budget = self.max_num_batched_tokens
        scheduled: dict[str, int] = {}
        for r in self.running:
            n = min(r.num_tokens - r.num_computed_tokens, budget)
            if n > 0:
                scheduled[r.request_id] = n
                budget -= n
        while self.waiting and len(self.running) < self.max_num_running_reqs and budget > 0:
            r = self.waiting[0]
            n = r.num_tokens - r.num_computed_tokens
            if n > budget:
                break
            self.waiting.pop(0)
            self.kv_cache_manager.allocate(r.request_id)
            r.status = RequestStatus.RUNNING
            self.running.append(r)
            scheduled[r.request_id] = n
            budget -= n
        for rid, n in scheduled.items():
            self.requests[rid].num_computed_tokens += n
        return SchedulerOutput(num_scheduled_tokens=scheduled)

    def update_from_output(self, scheduler_output: SchedulerOutput, model_runner_output) -> None:
        index = model_runner_output.req_id_to_index
        for rid in scheduler_output.num_scheduled_tokens:
            r = self.requests[rid]
            if rid not in index:
                continue
            for token in model_runner_output.sampled_token_ids[index[rid]]:
                r.output_token_ids.append(int(token))
                if int(token) == r.sampling_params.eos_token_id and not r.sampling_params.ignore_eos:
                    r.status = RequestStatus.FINISHED_STOPPED
                    break
                if r.num_output_tokens >= r.max_tokens:
                    r.status = RequestStatus.FINISHED_LENGTH_CAPPED
                    break
            if r.status in (RequestStatus.FINISHED_STOPPED, RequestStatus.FINISHED_LENGTH_CAPPED):
                self.running.remove(r)
                self.kv_cache_manager.release(rid)
