"""GPU parity of the multi-epoch cohort on one Qwen2.5-7B layer (bf16): a row
that keeps its generation across epochs, a row that is reused by a new
request under an incremented generation, and inactive rows, all through the
bridge call ``resident_epoch_execute`` (identity block table, row r owns
blocks 2r and 2r+1).

The trace is the reference's (run_multi_epoch_cohort.py:128-278,
verify_multi_epoch_cohort_result.py:28-63): A alone on row 0 (generation 1);
then A with B on row 1 (generation 2); B finishes after its budget; then A
with C, which reuses row 1 at generation 3.  K per epoch is the largest of
1, 2, 4, 8 within the configured maximum and every request's remaining
budget (scheduler.py:244-247).

Two variants:
* the reference's own: one-token prompts of the same token, budgets A 6,
  B 2, C 2, K at most 2 -- B's and C's tokens must equal A's first two, bit
  for bit (a reused row starts from a cleared block, so nothing of B leaks
  into C);
* seeded 2-5 token prompts (prefilled), budgets A 5, B 2, C 2-5.

Every epoch is compared with the oracle bridge over the oracle controller
(tokens, executed counts, generations, model calls, device status bit-exact,
teacher-forced where the top-2 margin is not decisive), the resident rows
exactly, A's key/value slots written in earlier epochs bit for bit against
their earlier contents, and the caches at the model tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cruise_amd.runtime import tiling_bytes
from oracle import bridge as obridge
from oracle.weights import generate_weights
from oracle.workloads import C2, identity_table
from parity import TeacherForcing, assert_close_rel, make_runtime, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C2
B = W.geometry.batch
BS = W.geometry.block_size
BPR = W.geometry.blocks_per_row
KVH = W.dims.num_kv_heads
D = W.dims.head_dim
EPOCH_CHOICES = (1, 2, 4, 8)


@pytest.fixture(scope="module")
def c2():
    dev = generate_weights(W.dims, W.seed, device="cuda")
    cpu = {k: v.cpu() for k, v in dev.items()}
    rt = make_runtime(W, dev)
    torch.cuda.synchronize()
    yield rt, cpu
    rt.close()


class Request:
    def __init__(self, name, prompt, budget):
        self.name = name
        self.prompt = list(prompt)
        self.budget = budget
        self.out: list[int] = []
        self.row = -1
        self.gen = 0
        self.position = len(prompt) - 1
        self.token = self.prompt[-1]

    @property
    def remaining(self):
        return self.budget - len(self.out)


def epoch_steps(max_steps, reqs):
    limit = min([max_steps] + [r.remaining for r in reqs])
    return max(k for k in EPOCH_CHOICES if k <= limit)


def read_kv(rt):
    k = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16)
    v = torch.zeros_like(k)
    rt.read_state("key_cache", k)
    rt.read_state("value_cache", v)
    shape = (W.dims.num_layers, W.geometry.physical_blocks * BS, KVH, D)
    return k.view(shape), v.view(shape)


def run_cohort(rt, cpu, prompts, budgets, max_steps):
    """Drive A, A+B, (B done), A+C ... until every request has its budget."""
    _, ctl = oracle_controller(W, cpu)
    zeros = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16, device="cuda")
    rt.write_state("key_cache", zeros)
    rt.write_state("value_cache", zeros)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))
    table = identity_table(B, BPR)
    reqs = {n: Request(n, prompts[n], budgets[n]) for n in "ABC"}
    next_gen = [1]
    rows_in_use: dict[int, Request] = {}
    trace = []
    written: dict[int, tuple] = {}  # row -> (slots of A written so far)

    def admit(req):
        free = min(r for r in range(B) if r not in rows_in_use)
        req.row = free
        req.gen = next_gen[0]
        next_gen[0] += 1
        rows_in_use[free] = req
        if len(req.prompt) > 1:  # prefill positions 0..L-2 and adopt the row
            rt.prefill(req.row, req.gen, req.prompt, table[req.row])
            ctl.prefill_row(req.row, req.gen, req.prompt, table[req.row])

    def epoch(label):
        active = [r for r in rows_in_use.values()]
        K = epoch_steps(max_steps, active)
        tok = [0] * B
        pos = [0] * B
        lens = [0] * B
        gens = [0] * B
        for r in active:
            tok[r.row], pos[r.row], lens[r.row], gens[r.row] = r.token, r.position, r.position + 1, r.gen
        eos = [W.eos] * B
        kv_before = read_kv(rt)
        out = rt.execute(len(active), K, tok, pos, lens, eos, gens)
        assert out.status == 0 and out.device_status == 0 and out.commit_state == 2, (label, out.status, out.device_status)
        assert out.feed_calls == 1 and out.fetch_calls == 1
        hist = np.full((8, B), -1, dtype=np.int64)
        for r in range(B):
            hist[: out.executed[r], r] = out.token_ids[r, : out.executed[r]]
        ctl.token_override = TeacherForcing(hist, rel_tol(W.dims))
        ref = obridge.execute(ctl, len(active), K, tok, pos, lens, eos, gens, tiling_bytes(), configured_eos=W.eos)
        assert not ctl.token_override.mismatches, (label, ctl.token_override.mismatches)
        np.testing.assert_array_equal(out.token_ids.reshape(-1), ref.token_ids, err_msg=label)
        np.testing.assert_array_equal(out.executed, ref.executed, err_msg=label)
        np.testing.assert_array_equal(out.row_generations, ref.row_generations, err_msg=label)
        assert out.model_calls == ref.model_calls == K and ref.device_status == 0
        assert list(out.row_generations) == gens
        rows = rt.resident_rows()
        np.testing.assert_array_equal(rows[0], ctl.resident_generation, err_msg=label)
        np.testing.assert_array_equal(rows[1], ctl.resident_token, err_msg=label)
        np.testing.assert_array_equal(rows[2], ctl.resident_position, err_msg=label)
        np.testing.assert_array_equal(rows[3], ctl.resident_length, err_msg=label)
        # slots A wrote before this epoch keep their bits
        a = reqs["A"]
        k_after, v_after = read_kv(rt)
        old = [table[a.row][p // BS] * BS + p % BS for p in range(a.position)]
        assert torch.equal(k_after[:, old], kv_before[0][:, old]), f"{label}: A's earlier keys changed"
        assert torch.equal(v_after[:, old], kv_before[1][:, old]), f"{label}: A's earlier values changed"
        for r in active:
            n = int(out.executed[r.row])
            toks = [int(t) for t in out.token_ids[r.row, :n]]
            r.out += toks
            r.token = toks[-1]
            r.position += n
            if toks[-1] == W.eos:  # finished at EOS before its budget
                r.budget = len(r.out)
        trace.append((label, {r.name: (r.row, r.gen) for r in active}, K, int(out.model_calls)))
        for r in active:
            if r.remaining == 0:
                del rows_in_use[r.row]

    admit(reqs["A"])
    epoch("epoch-1-a")
    admit(reqs["B"])
    epoch("epoch-2-a-b")
    while "B" in {r.name for r in rows_in_use.values()}:
        epoch("epoch-b-finishing")
    admit(reqs["C"])
    epoch("epoch-3-a-c")
    while rows_in_use:
        epoch("epoch-drain")
    k, v = read_kv(rt)
    assert_close_rel(k, ctl.resident_key.view_as(k), rel_tol(W.dims), "final resident keys")
    assert_close_rel(v, ctl.resident_value.view_as(v), rel_tol(W.dims), "final resident values")
    return reqs, trace


def test_reference_cohort_trace(c2):
    """One-token prompts of one token, K at most 2 (the reference's run)."""
    rt, cpu = c2
    token = 11690
    reqs, trace = run_cohort(rt, cpu, {"A": [token], "B": [token], "C": [token]}, {"A": 6, "B": 2, "C": 2}, 2)
    # verify_multi_epoch_cohort_result.py:29-63: rows and generations per epoch
    assert [t[1] for t in trace[:3]] == [{"A": (0, 1)}, {"A": (0, 1), "B": (1, 2)}, {"A": (0, 1), "C": (1, 3)}]
    assert [t[2] for t in trace[:3]] == [2, 2, 2]
    assert len(reqs["A"].out) == 6 and len(reqs["B"].out) == 2 and len(reqs["C"].out) == 2
    # the same prompt at a fresh generation gives A's first tokens, bit for bit
    assert reqs["B"].out == reqs["A"].out[:2] and reqs["C"].out == reqs["A"].out[:2]


def test_seeded_cohort_with_prefilled_prompts(c2):
    rt, cpu = c2
    rng = np.random.default_rng(W.seed + 4)
    prompts = {n: list(map(int, rng.integers(0, W.dims.vocab, size=int(rng.integers(2, 6))))) for n in "ABC"}
    budgets = {"A": 5, "B": 2, "C": int(rng.integers(2, 6))}
    print(f"[cohort] prompt lengths { {n: len(p) for n, p in prompts.items()} } budgets {budgets}", flush=True)
    reqs, trace = run_cohort(rt, cpu, prompts, budgets, 2)
    assert [t[1] for t in trace[:3]] == [{"A": (0, 1)}, {"A": (0, 1), "B": (1, 2)}, {"A": (0, 1), "C": (1, 3)}]
    for n in "ABC":
        assert len(reqs[n].out) == budgets[n]
