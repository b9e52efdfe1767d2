"""The C-ABI library and the host-side mirror, without a GPU.

* libresident_epoch.so loads and exports every entry point include/*.h
  declares, and the ctypes binding binds exactly those;
* the wire constants of include/resident_epoch_protocol.h equal the values
  their definitions give (native/resident_epoch_protocol.h:3-25 and the
  reference bridge's byte arithmetic);
* the device status / finish-reason enums equal the controller oracle's
  (CTRL:51-74);
* the host feed packing equals the declared byte layout (abi.py:18-76).
No test here calls into the GPU.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from cruise_amd import _lib, build
from cruise_amd.runtime import (
    EngineConfig,
    feed_layout,
    pack_feed,
    tiling_bytes,
    unpack_fetch,
)
from oracle import controller as ctl
from oracle.bridge import feed_bytes, fetch_bytes

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "resident_epoch.h"
PROTOCOL = ROOT / "include" / "resident_epoch_protocol.h"
LAYOUT = ROOT / "cruise_amd" / "csrc" / "re_layout.h"


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(resident_\w+)\s*\(", text))


def protocol_constants() -> dict[str, int]:
    out = {}
    for name, value in re.findall(r"#define\s+(CRUISE_\w+)\s+(0x[0-9A-Fa-f]+|\d+)(?:ULL)?\s*$", PROTOCOL.read_text(), flags=re.M):
        out[name] = int(value, 0)
    return out


@pytest.fixture(scope="module")
def lib():
    if not _lib.library_path().is_file():
        build.build()
    return _lib.load()


def test_library_exports_every_declared_entry_point(lib):
    declared = declared_functions()
    assert {"resident_epoch_create", "resident_epoch_execute", "resident_epoch_destroy"} <= declared
    for name in sorted(declared):
        assert hasattr(lib, name), f"{name} declared in {HEADER.name} but not exported"
    assert set(_lib.SIGNATURES) == declared


def test_protocol_constants():
    c = protocol_constants()
    layers, rows, block, kv_heads, head_dim, elem = 28, 4, 128, 4, 128, 2
    block_bytes = block * kv_heads * head_dim * elem
    assert c["CRUISE_RESIDENT_KV_BLOCK_BYTES"] == block_bytes
    # K and V caches of the imported rows' first blocks (CTRL:25-26)
    payload = 2 * layers * rows * block_bytes
    assert c["CRUISE_RESIDENT_IMPORT_PAYLOAD_BYTES"] == payload
    # the import feed drops slot_mapping (BRIDGE:53-62, CTRL:217-221)
    assert c["CRUISE_RESIDENT_IMPORT_INPUT_BYTES"] == payload + feed_bytes(4, 2) - 4 * rows
    assert c["CRUISE_RESIDENT_IMPORT_GRAPH_FLAG"] == ctl.IMPORT_GRAPH_FLAG
    assert (c["CRUISE_EPOCH_PREPARED"], c["CRUISE_EPOCH_EXECUTING"], c["CRUISE_EPOCH_COMMITTED"]) == (0, 1, 2)
    assert c["CRUISE_RESIDENT_TRANSFER_MAGIC"].to_bytes(8, "big") == b"CRUISEKV"
    assert c["CRUISE_RESIDENT_IPC_METADATA_MAGIC"].to_bytes(8, "big") == b"CRUISEIP"


def test_device_enums_match_controller_oracle():
    text = LAYOUT.read_text()
    values = {name: int(v) for name, v in re.findall(r"\b(k(?:Status|Finish)\w+)\s*=\s*(\d+)", text)}
    expect = {
        "kStatusOk": ctl.STATUS_OK,
        "kStatusInvalidMetadata": ctl.STATUS_INVALID_METADATA,
        "kStatusCapacityExceeded": ctl.STATUS_CAPACITY_EXCEEDED,
        "kStatusInvalidBlockTable": ctl.STATUS_INVALID_BLOCK_TABLE,
        "kStatusSlotMismatch": ctl.STATUS_SLOT_MISMATCH,
        "kStatusUnsupportedSampling": ctl.STATUS_UNSUPPORTED_SAMPLING,
        "kStatusUnsupportedGraph": ctl.STATUS_UNSUPPORTED_GRAPH,
        "kStatusModelError": ctl.STATUS_MODEL_ERROR,
        "kStatusInvalidModelOutput": ctl.STATUS_INVALID_MODEL_OUTPUT,
        "kStatusNonFiniteLogits": ctl.STATUS_NON_FINITE_LOGITS,
        "kStatusPositionProgress": ctl.STATUS_POSITION_PROGRESS,
        "kStatusAllocationFailure": ctl.STATUS_ALLOCATION_FAILURE,
        "kStatusResidentContinuity": ctl.STATUS_RESIDENT_CONTINUITY,
        "kFinishNone": ctl.FINISH_NONE,
        "kFinishEos": ctl.FINISH_EOS,
        "kFinishMaxSteps": ctl.FINISH_MAX_STEPS,
        "kFinishFallback": ctl.FINISH_FALLBACK,
        "kFinishEmpty": ctl.FINISH_EMPTY,
        "kFinishAlreadyFinished": ctl.FINISH_ALREADY,
    }
    assert values == expect


def test_feed_layout_matches_declared_bytes():
    lay = feed_layout(4, 2)
    assert lay["_total"][1] == feed_bytes(4, 2) == 260
    # ABI order (BRIDGE:53-62): token, position, length, slot, active, table, tiling, control
    order = [k for k in lay if not k.startswith("_")]
    assert order == ["token", "position", "sequence_length", "slot_mapping", "active_mask", "block_table", "tiling", "control"]
    offsets = [lay[k][0] for k in order]
    assert offsets == sorted(offsets) and offsets[0] == 0
    imp = feed_layout(4, 2, importing=True, payload_bytes=protocol_constants()["CRUISE_RESIDENT_IMPORT_PAYLOAD_BYTES"])
    assert imp["_total"][1] == protocol_constants()["CRUISE_RESIDENT_IMPORT_INPUT_BYTES"]
    assert "slot_mapping" not in imp and imp["payload"][0] == 0


def test_pack_feed_round_trip():
    tok = np.array([1, 2, 3, 4], dtype=np.int64)
    pos = np.array([5, 6, 7, 8], dtype=np.int64)
    ln = (pos + 1).astype(np.int32)
    slot = np.array([9, 10, 11, 12], dtype=np.int32)
    act = np.array([1, 0, 1, 0], dtype=np.int32)
    table = np.arange(8, dtype=np.int32)
    control = np.arange(11, dtype=np.int32)
    raw = pack_feed(tok, pos, ln, slot, act, table, tiling_bytes(), control)
    lay = feed_layout(4, 2)
    assert len(raw) == lay["_total"][1]

    def field(name, dtype):
        off, size = lay[name]
        return np.frombuffer(raw[off : off + size], dtype=dtype)

    assert np.array_equal(field("token", "<i8"), tok) and np.array_equal(field("position", "<i8"), pos)
    assert np.array_equal(field("slot_mapping", "<i4"), slot) and np.array_equal(field("block_table", "<i4"), table)
    assert np.array_equal(field("control", "<i4"), control)
    assert bytes(field("tiling", np.uint8)) == tiling_bytes()


def test_tiling_record_is_the_reference_72_bytes():
    # batched_decoder_step.py:36 (18 little-endian uint32 words)
    words = np.frombuffer(tiling_bytes(), dtype="<u4")
    assert len(tiling_bytes()) == 72
    assert list(words[:4]) == [28, 1, 128, 8]


def test_unpack_fetch():
    hist = np.arange(32, dtype=np.int64).reshape(8, 4)
    control = np.arange(28, dtype=np.int32)
    raw = hist.tobytes() + control.tobytes()
    assert len(raw) == fetch_bytes(4) == 368
    h, c = unpack_fetch(raw, 4)
    assert np.array_equal(h, hist) and np.array_equal(c, control)


def test_engine_config_json_keys():
    import json

    cfg = json.loads(EngineConfig().to_json())
    assert set(cfg) == {"model", "engine", "weights"}
    assert cfg["model"]["hidden"] == 3584 and cfg["engine"]["batch"] == 4
    assert cfg["engine"]["configured_eos"] == 151645


def test_gemm_entry_point_rejects_bad_arguments_before_any_device_work(lib):
    # every refusal below happens before the library touches a device
    p = ctypes.c_void_p(16)  # never dereferenced: the checks fail first
    null = None
    f = lib.resident_epoch_gemm
    assert f(null, p, null, null, p, 8, 8, 64, 0, 2) == -1  # no A
    assert f(p, null, null, null, p, 8, 8, 64, 0, 2) == -1  # no W
    assert f(p, p, null, null, null, 8, 8, 64, 0, 2) == -1  # no out
    assert f(p, p, null, null, p, -1, 8, 64, 0, 2) == -1  # M < 0
    assert f(p, p, null, null, p, 8, 0, 64, 0, 2) == -1  # N = 0
    assert f(p, p, null, null, p, 8, 8, 0, 0, 2) == -1  # K = 0
    assert f(p, p, null, null, p, 8, 8, 64, 3, 2) == -1  # no such epilogue
    assert f(p, p, null, null, p, 8, 8, 64, 0, 3) == -1  # element size
    assert f(p, p, null, null, p, 8, 8, 64, 2, 2) == -1  # SwiGLU without the up rows
    assert f(p, p, null, ctypes.c_void_p(20), p, 8, 8, 64, 0, 2) == -1  # bias not 8-byte aligned
