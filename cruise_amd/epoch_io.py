"""The fixed-shape exchange of one epoch with a native engine.

Both native engines -- the sidecar client (sidecar_backend.py) and the
in-process library (ctypes_backend.py) -- hand the engine the same per-row
arrays and receive the same counters back; they differ only in transport.
This module is that shared part: ``EpochFeed`` is a plan laid out on the
four graph rows (the inputs of resident_epoch_execute, BRIDGE.h:24-45), and
``EpochFetch`` is what one call returned, decoded into the backend's
NativeEpochOutput / NativeWarmupOutput with every consistency check a
transport-independent client can make.

Row layout of a feed (resident_epoch_bridge.cpp:424-560): a row without a
request carries token 0, position 0, length 0, generation 0 and the default
EOS 151645.  Token history comes back row-major, 8 slots per row.  The
warm-up is one decoder step of row 0 with token 11690 under the reserved
generation 2^31-1 (sidecar_backend.py:218-272).
"""
from __future__ import annotations

from dataclasses import dataclass

from .backend import NativeEpochOutput, NativeWarmupOutput
from .contract import EpochCommitState, ResidentEpochExecutionError, ResidentEpochPlan

ROWS = 4
MAX_EPOCH_STEPS = 8
DEFAULT_EOS = 151645
WARMUP_TOKEN = 11690
WARMUP_GENERATION = 2**31 - 1


@dataclass(frozen=True)
class EpochFeed:
    """One epoch's inputs, one value per graph row."""

    request_count: int
    max_steps: int
    tokens: tuple[int, ...]
    positions: tuple[int, ...]
    lengths: tuple[int, ...]
    eos: tuple[int, ...]
    generations: tuple[int, ...]

    @classmethod
    def from_plan(cls, plan: ResidentEpochPlan) -> "EpochFeed":
        if plan.graph_batch_size != ROWS:
            raise ValueError(f"the native engine runs a {ROWS}-row graph, the plan has {plan.graph_batch_size} rows")
        columns = {"token_id": [0] * ROWS, "position": [0] * ROWS, "sequence_length": [0] * ROWS,
                   "eos_token_id": [DEFAULT_EOS] * ROWS}
        for request in plan.requests:
            for name, column in columns.items():
                column[request.row] = int(getattr(request, name))
        return cls(len(plan.requests), plan.max_steps, tuple(columns["token_id"]), tuple(columns["position"]),
                   tuple(columns["sequence_length"]), tuple(columns["eos_token_id"]), tuple(plan.row_generations))

    @classmethod
    def warm_up(cls, token: int = WARMUP_TOKEN, eos: int = DEFAULT_EOS) -> "EpochFeed":
        """One step of row 0 under the reserved generation; a model with a
        smaller vocabulary passes a token and EOS of its own."""
        return cls(1, 1, (token, 0, 0, 0), (0, 0, 0, 0), (1, 0, 0, 0), (eos,) * ROWS, (WARMUP_GENERATION, 0, 0, 0))

    @classmethod
    def empty(cls) -> "EpochFeed":
        """The all-zero feed a control record without an epoch carries."""
        zeros = (0,) * ROWS
        return cls(0, 0, zeros, zeros, zeros, zeros, zeros)


def import_mask(plan: ResidentEpochPlan) -> int:
    """Bit r set for every row whose KV the plan imports."""
    return sum(1 << r.row for r in plan.requests if r.kv_import_required)


def check_transfer(plan: ResidentEpochPlan, mask: int, generations, what: str) -> None:
    """A KV transfer must cover exactly the plan's importing rows under
    their generations (sidecar_backend.py:303-343)."""
    if mask != import_mask(plan):
        raise ValueError(f"{what}: import mask {mask:#x} differs from the plan's {import_mask(plan):#x}")
    expected = [0] * ROWS
    for request in plan.requests:
        if request.kv_import_required:
            expected[request.row] = request.generation
    if tuple(generations) != tuple(expected):
        raise ValueError(f"{what}: row generations {tuple(generations)} differ from the plan's {tuple(expected)}")


def decode_commit_state(code: int, source: str) -> EpochCommitState:
    """A commit-state code from the engine; an unknown code means nothing
    proves how far the epoch got, which is the EXECUTING state."""
    try:
        return EpochCommitState(code)
    except ValueError:
        raise ResidentEpochExecutionError(f"{source} reported commit state {code}, which does not exist",
                                          commit_state=EpochCommitState.EXECUTING) from None


@dataclass(frozen=True)
class EpochFetch:
    """What one engine call returned.  ``transport_status`` is the call's own
    status (resident_epoch_execute's return value, or the server's transport
    status); ``device_status`` is the controller's fallback code (0 or
    201-212)."""

    transport_status: int
    device_status: int
    model_calls: int
    feed_calls: int
    fetch_calls: int
    commit_code: int
    checksum: int
    wall_us: int
    native_cpu_us: int
    declared_input_bytes: int
    declared_output_bytes: int
    executed: tuple[int, ...]
    generations: tuple[int, ...]
    history: tuple[int, ...]
    source: str = "native engine"

    def commit_state(self) -> EpochCommitState:
        return decode_commit_state(self.commit_code, self.source)

    def raise_for_transport(self) -> EpochCommitState:
        """The commit state, after turning a failed call into an execution
        error that carries it."""
        state = self.commit_state()
        if self.transport_status != 0:
            raise ResidentEpochExecutionError(f"{self.source} call failed with status {self.transport_status}",
                                              commit_state=state, status=self.transport_status)
        return state

    def row_tokens(self, row: int, count: int) -> list[int]:
        start = row * MAX_EPOCH_STEPS
        return [int(t) for t in self.history[start:start + count]]

    def native_output(self, plan: ResidentEpochPlan, transfer_mode: str = "none") -> NativeEpochOutput:
        state = self.raise_for_transport()
        tokens = {}
        for request in plan.requests:
            count = self.executed[request.row]
            if not 0 <= count <= plan.max_steps:
                raise ResidentEpochExecutionError(
                    f"{self.source} reports {count} executed steps on row {request.row} of a {plan.max_steps}-step "
                    "epoch", commit_state=state)
            tokens[request.req_id] = self.row_tokens(request.row, count)
        return NativeEpochOutput(
            status=self.device_status, model_calls=self.model_calls, token_ids=tokens,
            row_generations=tuple(self.generations), commit_state=state, feed_calls=self.feed_calls,
            fetch_calls=self.fetch_calls, wall_us=self.wall_us, native_cpu_us=self.native_cpu_us,
            declared_input_bytes=self.declared_input_bytes, declared_output_bytes=self.declared_output_bytes,
            kv_imported=transfer_mode != "none", kv_import_checksum=self.checksum & 0xFFFFFFFF,
            kv_transfer_mode=transfer_mode,
        )

    def warmup_output(self) -> NativeWarmupOutput:
        state = self.raise_for_transport()
        if tuple(self.executed) != (1, 0, 0, 0):
            raise RuntimeError(f"the warm-up ran {tuple(self.executed)} steps per row instead of one step on row 0")
        if tuple(self.generations) != (WARMUP_GENERATION, 0, 0, 0):
            raise RuntimeError(f"the warm-up acknowledged generations {tuple(self.generations)}")
        return NativeWarmupOutput(
            status=self.device_status, model_calls=self.model_calls, feed_calls=self.feed_calls,
            fetch_calls=self.fetch_calls, commit_state=state, wall_us=self.wall_us,
            native_cpu_us=self.native_cpu_us, declared_input_bytes=self.declared_input_bytes,
            declared_output_bytes=self.declared_output_bytes,
        )
