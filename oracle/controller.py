"""CPU restatement of the device epoch controller ``G4cB4ResidentEpoch::Proc``.

Oracle (test infrastructure only).  Restates
controller/g4c_b4_resident_epoch.cpp ("CTRL") with the B=4 / capacity-8 /
8-block constants (CTRL:13-38) turned into parameters:

* ``compute_slot``      -- CTRL:84-97
* ``argmax_finite``     -- CTRL:99-119
* ``adler32_update``    -- CTRL:149-163
* ``EpochController.proc`` -- CTRL:177-622 (validation 335-385, import
  387-446, generation continuity and row clear 448-471, K-step loop 485-590,
  finish reasons 592-597, resident save 599-614, ``emit`` 296-324)

Decisions recorded against CTRL:

* N1 capacity is a parameter (CTRL:18 hard-codes 8).
* N2 the row clear and the import follow the row's block-table entries; CTRL
  clears/imports blocks ``row*BPR ..`` (CTRL:140-142, 415-418).  Both agree on
  the identity table ``[[0,1],[2,3],...]`` the bridge always feeds
  (native/resident_epoch_bridge.cpp:524-526).
* The model is any callable with the decoder ABI (``OracleDecoder.forward``).
  As in CTRL the step's output caches become the resident caches only when the
  epoch completes (CTRL:583-584, 599-600): a fallback inside the loop leaves
  the pre-epoch caches resident.

Parity pinning: the integer logic is pinned by known-answer cases derived by
hand from CTRL's closed forms (every fallback code forced from the feed,
EOS/max-step reasons, generation continuity, history layout), by the
reference's own contract/cohort expectations and by a pure-brute-force
recomputation of the history from the decoder's logits
(tests/test_oracle_controller.py).  ``argmax_finite`` is pinned against
``numpy.argmax`` first-occurrence semantics plus NaN/Inf brute force,
``adler32_update`` against ``zlib.adler32``.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable

import numpy as np
import torch

# Finish reasons (CTRL:51-58) and device statuses (CTRL:60-74).
FINISH_NONE, FINISH_EOS, FINISH_MAX_STEPS, FINISH_FALLBACK, FINISH_EMPTY, FINISH_ALREADY = 0, 1, 2, 3, 4, 5
STATUS_OK = 0
STATUS_INVALID_METADATA = 201
STATUS_CAPACITY_EXCEEDED = 202
STATUS_INVALID_BLOCK_TABLE = 203
STATUS_SLOT_MISMATCH = 204
STATUS_UNSUPPORTED_SAMPLING = 205
STATUS_UNSUPPORTED_GRAPH = 206
STATUS_MODEL_ERROR = 207
STATUS_INVALID_MODEL_OUTPUT = 208
STATUS_NON_FINITE_LOGITS = 209
STATUS_POSITION_PROGRESS = 210
STATUS_ALLOCATION_FAILURE = 211
STATUS_RESIDENT_CONTINUITY = 212

MAX_EPOCH_STEPS = 8  # CTRL:17
IMPORT_GRAPH_FLAG = 0x100  # CTRL:27


def control_input_elements(batch: int) -> int:
    """CTRL:28: ``[K, eos[B], sampling, variant, gen[B]]``."""
    return 1 + batch + 2 + batch


def control_output_elements(batch: int) -> int:
    """CTRL:29."""
    return 6 + 4 * batch + 2 + batch


@dataclass(frozen=True)
class ControllerGeometry:
    batch: int
    capacity: int
    physical_blocks: int
    blocks_per_row: int
    block_size: int
    vocab: int
    num_layers: int

    # Output control offsets (CTRL:30-38).
    @property
    def eos_off(self) -> int:
        return 6

    @property
    def initial_active_off(self) -> int:
        return 6 + self.batch

    @property
    def executed_off(self) -> int:
        return 6 + 2 * self.batch

    @property
    def reason_off(self) -> int:
        return 6 + 3 * self.batch

    @property
    def initial_count_off(self) -> int:
        return 6 + 4 * self.batch

    @property
    def final_count_off(self) -> int:
        return 6 + 4 * self.batch + 1

    @property
    def generation_off(self) -> int:
        return 6 + 4 * self.batch + 2


def compute_slot(g: ControllerGeometry, block_table, request: int, position: int) -> int:
    """CTRL:84-97."""
    if request < 0 or request >= g.batch or position < 0 or position >= g.capacity:
        return -1
    logical_block = position // g.block_size
    offset = position % g.block_size
    if logical_block >= g.blocks_per_row:
        return -1
    physical = int(block_table[request * g.blocks_per_row + logical_block])
    if physical < 0 or physical >= g.physical_blocks:
        return -1
    return physical * g.block_size + offset


def argmax_finite(logits_row: np.ndarray) -> int | None:
    """CTRL:99-119: first index of the strict maximum; ``None`` if any value is
    NaN or infinite."""
    row = np.asarray(logits_row, dtype=np.float32)
    if not np.all(np.isfinite(row)):
        return None
    # The scan keeps the first index of the strict maximum; numpy's argmax
    # returns the first occurrence of the maximum.
    return int(np.argmax(row))


def adler32_update(data: bytes, first: int, second: int) -> tuple[int, int]:
    """CTRL:149-163 (chunks of 5552 bytes, modulus 65521)."""
    mod = 65521
    view = np.frombuffer(data, dtype=np.uint8)
    pos = 0
    while pos < len(view):
        chunk = view[pos : pos + 5552].astype(np.int64)
        # first_i = first + sum(data[:i+1]); second += sum_i first_i
        prefix = np.cumsum(chunk)
        second = (second + first * len(chunk) + int(prefix.sum())) % mod
        first = (first + int(prefix[-1])) % mod
        pos += len(chunk)
    return first, second


@dataclass
class EpochFeed:
    """The 8-input epoch ABI (CTRL:40-49; native/resident_epoch_bridge.cpp:53-62)."""

    token: np.ndarray  # int64 [B]
    position: np.ndarray  # int64 [B]
    sequence_length: np.ndarray  # int32 [B]
    slot_mapping: np.ndarray  # int32 [B]
    active_mask: np.ndarray  # int32 [B]
    block_table: np.ndarray  # int32 [B * BPR]
    tiling: bytes  # 72 bytes
    control: np.ndarray  # int32 [3 + 2B]
    import_payload: bytes | None = None  # present only in import mode


@dataclass
class EpochFetch:
    """The 2-output epoch ABI: token history [8, B] and control [6+4B+2+B]."""

    history: np.ndarray  # int64 [8, B]
    control: np.ndarray  # int32


Model = Callable[..., tuple]


@dataclass
class EpochController:
    """Resident state plus ``Proc`` (CTRL:166-632)."""

    geometry: ControllerGeometry
    model: Model
    cache_shape: tuple[int, ...]
    cache_dtype: torch.dtype
    resident_key: torch.Tensor | None = None
    resident_value: torch.Tensor | None = None
    resident_generation: list = field(default_factory=list)
    resident_token: list = field(default_factory=list)
    resident_position: list = field(default_factory=list)
    resident_length: list = field(default_factory=list)
    resident_valid: list = field(default_factory=list)
    logits_trace: list = field(default_factory=list)
    token_override: Callable | None = None

    def __post_init__(self) -> None:
        B = self.geometry.batch
        # Init (CTRL:168-175).
        self.resident_generation = [0] * B
        self.resident_token = [0] * B
        self.resident_position = [0] * B
        self.resident_length = [0] * B
        self.resident_valid = [0] * B

    # -- helpers -------------------------------------------------------------
    def ensure_caches(self) -> None:
        if self.resident_key is None:  # CTRL:247-262
            self.resident_key = torch.zeros(self.cache_shape, dtype=self.cache_dtype)
            self.resident_value = torch.zeros(self.cache_shape, dtype=self.cache_dtype)

    def prefill_row(self, row: int, generation: int, prompt: list[int], table_row) -> None:
        """Teacher-forced prefill of one row and its adoption as resident state.

        Stands in for the stock-vLLM prefill plus KV import the reference uses
        to hand a prompt's KV to the device (CTRL:387-429 sets the resident
        record from the feed after the copy): clear the row's blocks, run the
        decoder at positions 0..L-2 with only this row active, then record
        generation, token prompt[L-1], position L-1, length L.

        Pinned by tests/test_oracle_prefill.py: the written K (post-RoPE) and
        V of every layer against HF ``Qwen2ForCausalLM`` eager's DynamicCache
        after the same L-1 tokens, the row's later slots zero, every other
        block untouched, and the resident record exact; planted mistakes in
        ``_prefill_positions`` and ``_clear_row_blocks`` fail it.
        """
        g = self.geometry
        B = g.batch
        self.ensure_caches()
        table = np.zeros((B, g.blocks_per_row), dtype=np.int32)
        table[row] = np.asarray(table_row, dtype=np.int32)
        self._clear_row_blocks(table[row])
        tiling = torch.zeros(72, dtype=torch.uint8)
        for p in self._prefill_positions(prompt):
            tok = np.zeros((B, 1), dtype=np.int64)
            pos = np.zeros(B, dtype=np.int64)
            length = np.zeros((B, 1), dtype=np.int32)
            slot = np.full(B, -1, dtype=np.int32)
            act = np.zeros(B, dtype=np.int32)
            tok[row, 0] = prompt[p]
            pos[row] = p
            length[row, 0] = p + 1
            slot[row] = int(table[row, p // g.block_size]) * g.block_size + p % g.block_size
            act[row] = 1
            self.model(
                torch.from_numpy(tok),
                torch.from_numpy(pos),
                torch.from_numpy(length),
                torch.from_numpy(table),
                torch.from_numpy(slot),
                self.resident_key,
                self.resident_value,
                tiling,
                torch.from_numpy(act),
                inplace=True,
            )
        self.resident_generation[row] = generation
        self.resident_token[row] = int(prompt[-1])
        self.resident_position[row] = len(prompt) - 1
        self.resident_length[row] = len(prompt)
        self.resident_valid[row] = 1

    @staticmethod
    def _prefill_positions(prompt: list[int]) -> range:
        """Positions a prompt of length L writes before the epoch: 0..L-2
        (the last prompt token is the epoch's first input, CTRL:458-463)."""
        return range(len(prompt) - 1)

    def _clear_row_blocks(self, table_row) -> None:
        """Zero every block the row owns in both caches (ClearCacheRow,
        CTRL:129-147, before the import copy at CTRL:402-405)."""
        for block in table_row:
            self.resident_key[:, int(block)].zero_()
            self.resident_value[:, int(block)].zero_()

    def _clear_row(self, cache: torch.Tensor, block_table, row: int) -> None:
        """ClearCacheRow (CTRL:129-147), following the row's table entries (N2)."""
        g = self.geometry
        for local in range(g.blocks_per_row):
            block = int(block_table[row * g.blocks_per_row + local])
            cache[:, block].zero_()

    def proc(self, feed: EpochFeed) -> EpochFetch:
        g = self.geometry
        B = g.batch
        history = np.full((MAX_EPOCH_STEPS, B), -1, dtype=np.int64)  # CTRL:194-198
        control = np.zeros(control_output_elements(B), dtype=np.int32)  # CTRL:199-202
        ctl_in = np.asarray(feed.control, dtype=np.int32)
        if ctl_in.shape != (control_input_elements(B),):
            raise ValueError("invalid control ABI")  # CTRL:204-208 (FLOW_FUNC_FAILED)
        encoded_variant = int(ctl_in[2 + B])
        importing = (encoded_variant & IMPORT_GRAPH_FLAG) != 0  # CTRL:211-217
        import_mask = encoded_variant & (IMPORT_GRAPH_FLAG - 1) if importing else 0
        graph_variant = encoded_variant & ~(IMPORT_GRAPH_FLAG | 0xF) if importing else encoded_variant

        token = np.asarray(feed.token, dtype=np.int64).reshape(B)
        position = np.asarray(feed.position, dtype=np.int64).reshape(B)
        length = np.asarray(feed.sequence_length, dtype=np.int32).reshape(B)
        active = np.asarray(feed.active_mask, dtype=np.int32).reshape(B)
        table = np.asarray(feed.block_table, dtype=np.int32).reshape(B * g.blocks_per_row)
        if len(feed.tiling) != 72:
            raise ValueError("invalid tensor ABI")  # CTRL:230-245
        if importing:
            slot = np.array([compute_slot(g, table, r, int(position[r])) for r in range(B)], dtype=np.int32)
        else:
            slot = np.asarray(feed.slot_mapping, dtype=np.int32).reshape(B).copy()

        if self.resident_key is None:  # CTRL:247-262
            self.resident_key = torch.zeros(self.cache_shape, dtype=self.cache_dtype)
            self.resident_value = torch.zeros(self.cache_shape, dtype=self.cache_dtype)

        max_steps = int(ctl_in[0])
        eos = [int(ctl_in[1 + r]) for r in range(B)]
        sampling = int(ctl_in[1 + B])
        row_generation = [int(ctl_in[3 + B + r]) for r in range(B)]
        executed = [0] * B
        reason = [FINISH_NONE] * B
        state = {"model_calls": 0, "checksum": 0}

        def emit(status: int, final_active) -> EpochFetch:  # CTRL:296-324
            control[0] = max_steps
            control[1] = sampling
            control[2] = graph_variant
            control[3] = status
            control[4] = state["model_calls"]
            control[5] = np.int32(np.uint32(state["checksum"]).view(np.int32)) if importing else (0 if status == STATUS_OK else 1)
            for r in range(B):
                control[g.eos_off + r] = eos[r]
                control[g.initial_active_off + r] = active[r]
                control[g.executed_off + r] = executed[r]
                control[g.reason_off + r] = reason[r]
                control[g.generation_off + r] = row_generation[r] if active[r] == 1 else 0
            control[g.initial_count_off] = int(np.count_nonzero(active))
            control[g.final_count_off] = int(np.count_nonzero(np.asarray(final_active)))
            return EpochFetch(history=history, control=control)

        def fallback(status: int) -> EpochFetch:  # CTRL:326-333
            for r in range(B):
                reason[r] = FINISH_FALLBACK
            return emit(status, active)

        # Validation, first match wins (CTRL:335-385).
        if max_steps < 1 or max_steps > MAX_EPOCH_STEPS or sampling != 0 or graph_variant != 0:
            if sampling != 0:
                return fallback(STATUS_UNSUPPORTED_SAMPLING)
            if graph_variant != 0:
                return fallback(STATUS_UNSUPPORTED_GRAPH)
            return fallback(STATUS_INVALID_METADATA)
        for r in range(B):
            if eos[r] < 0 or eos[r] >= g.vocab:
                return fallback(STATUS_INVALID_METADATA)
        seen = set()
        for block in table:
            block = int(block)
            if block < 0 or block >= g.physical_blocks or block in seen:
                return fallback(STATUS_INVALID_BLOCK_TABLE)
            seen.add(block)
        for r in range(B):
            if (
                active[r] not in (0, 1)
                or token[r] < 0
                or token[r] >= g.vocab
                or position[r] < 0
                or position[r] >= g.capacity
            ):
                return fallback(STATUS_INVALID_METADATA)
            if active[r] == 1:
                if row_generation[r] <= 0:
                    return fallback(STATUS_INVALID_METADATA)
                if length[r] != position[r] + 1:
                    return fallback(STATUS_INVALID_METADATA)
                if position[r] + max_steps > g.capacity:
                    return fallback(STATUS_CAPACITY_EXCEEDED)
            elif length[r] == 0:
                if row_generation[r] != 0:
                    return fallback(STATUS_INVALID_METADATA)
                reason[r] = FINISH_EMPTY
            elif length[r] == position[r] + 1:
                reason[r] = FINISH_ALREADY
            else:
                return fallback(STATUS_INVALID_METADATA)
            if compute_slot(g, table, r, int(position[r])) != slot[r]:
                return fallback(STATUS_SLOT_MISMATCH)

        if importing:  # CTRL:387-446
            if import_mask <= 0 or import_mask >= (1 << B):
                return fallback(STATUS_INVALID_METADATA)
            payload = feed.import_payload
            block_elems = g.block_size * self.cache_shape[3] * self.cache_shape[4]
            per_cache = g.num_layers * B * block_elems
            src = torch.frombuffer(bytearray(payload), dtype=self.cache_dtype)
            src_k = src[:per_cache].view(g.num_layers, B, g.block_size, self.cache_shape[3], self.cache_shape[4])
            src_v = src[per_cache : 2 * per_cache].view_as(src_k)
            for r in range(B):
                if (import_mask & (1 << r)) == 0:
                    continue
                if active[r] != 1 or row_generation[r] <= 0:
                    return fallback(STATUS_INVALID_METADATA)
                self._clear_row(self.resident_key, table, r)
                self._clear_row(self.resident_value, table, r)
                dest = int(table[r * g.blocks_per_row])
                self.resident_key[:, dest] = src_k[:, r]
                self.resident_value[:, dest] = src_v[:, r]
                self.resident_generation[r] = row_generation[r]
                self.resident_token[r] = int(token[r])
                self.resident_position[r] = int(position[r])
                self.resident_length[r] = int(length[r])
                self.resident_valid[r] = 1
            first, second = 1, 0
            for cache in (self.resident_key, self.resident_value):
                for layer in range(g.num_layers):
                    for r in range(B):
                        if (import_mask & (1 << r)) == 0:
                            continue
                        dest = int(table[r * g.blocks_per_row])
                        raw = cache[layer, dest].contiguous().view(torch.uint8).numpy().tobytes()
                        first, second = adler32_update(raw, first, second)
            state["checksum"] = ((second << 16) | first) & 0xFFFFFFFF

        new_generation = [0] * B  # CTRL:448-471
        for r in range(B):
            if active[r] == 0:
                continue
            if self.resident_generation[r] == row_generation[r]:
                if (
                    self.resident_valid[r] == 0
                    or self.resident_token[r] != token[r]
                    or self.resident_position[r] != position[r]
                    or self.resident_length[r] != length[r]
                ):
                    return fallback(STATUS_RESIDENT_CONTINUITY)
            else:
                if position[r] != 0 or length[r] != 1:
                    return fallback(STATUS_RESIDENT_CONTINUITY)
                new_generation[r] = 1
        for r in range(B):
            if new_generation[r]:
                self._clear_row(self.resident_key, table, r)
                self._clear_row(self.resident_value, table, r)

        # K-step loop (CTRL:473-590).  The step works on copies so the
        # resident caches change only on success (CTRL:583-584, 599-600).
        cur_token = token.copy()
        cur_position = position.copy()
        cur_length = length.copy()
        cur_slot = slot.copy()
        cur_active = active.copy()
        cur_key = self.resident_key.clone()
        cur_value = self.resident_value.clone()
        tiling = torch.frombuffer(bytearray(feed.tiling), dtype=torch.uint8)
        table_t = torch.from_numpy(table.reshape(B, g.blocks_per_row).copy())
        self.logits_trace = []
        while state["model_calls"] < max_steps:
            if np.count_nonzero(cur_active) == 0:
                break
            logits, cur_key, cur_value, next_position = self.model(
                torch.from_numpy(cur_token.reshape(B, 1).copy()),
                torch.from_numpy(cur_position.copy()),
                torch.from_numpy(cur_length.reshape(B, 1).copy()),
                table_t,
                torch.from_numpy(cur_slot.copy()),
                cur_key,
                cur_value,
                tiling,
                torch.from_numpy(cur_active.copy()),
            )
            state["model_calls"] += 1
            logits_np = logits.reshape(B, -1).float().numpy()
            self.logits_trace.append(logits_np.copy())
            next_pos = next_position.numpy().astype(np.int64)
            next_token = cur_token.copy()
            next_length = cur_length.copy()
            next_slot = cur_slot.copy()
            next_active = cur_active.copy()
            for r in range(B):
                if cur_active[r] == 0:
                    if next_pos[r] != cur_position[r]:
                        return fallback(STATUS_POSITION_PROGRESS)
                    continue
                generated = argmax_finite(logits_np[r])
                if generated is None:
                    return fallback(STATUS_NON_FINITE_LOGITS)
                if self.token_override is not None:
                    generated = self.token_override(state["model_calls"] - 1, r, generated, logits_np[r])
                if next_pos[r] != cur_position[r] + 1:
                    return fallback(STATUS_POSITION_PROGRESS)
                history[state["model_calls"] - 1, r] = generated
                executed[r] += 1
                cur_position[r] = next_pos[r]
                next_token[r] = generated
                next_length[r] = cur_position[r] + 1
                if cur_position[r] == g.capacity:
                    next_slot[r] = -1
                else:
                    s = compute_slot(g, table, r, int(cur_position[r]))
                    if s < 0:
                        return fallback(STATUS_CAPACITY_EXCEEDED)
                    next_slot[r] = s
                if generated == eos[r]:
                    next_active[r] = 0
                    reason[r] = FINISH_EOS
            cur_position = next_pos.copy()
            cur_token = next_token
            cur_length = next_length
            cur_slot = next_slot
            cur_active = next_active

        for r in range(B):  # CTRL:592-597
            if active[r] == 1 and reason[r] == FINISH_NONE:
                reason[r] = FINISH_MAX_STEPS
        self.resident_key = cur_key  # CTRL:599-614
        self.resident_value = cur_value
        for r in range(B):
            if active[r] == 0:
                continue
            self.resident_generation[r] = row_generation[r]
            self.resident_token[r] = int(cur_token[r])
            self.resident_position[r] = int(cur_position[r])
            self.resident_length[r] = int(cur_length[r])
            self.resident_valid[r] = 1
        return emit(STATUS_OK, cur_active)

