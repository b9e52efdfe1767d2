"""Child process of tests/test_gpu_ipc_qwen7b.py: a worker that owns stock
paged KV caches on the GPU and exports them for a device-IPC import.

It allocates one [blocks, block_size, kv_heads, head_dim] bf16 tensor per
layer and cache (each its own allocation), fills them from a seed, builds
the IPC record with ``cruise_amd.kv_transfer.capture_kv_device_transfer``
for the rows and blocks it is given, writes the host-path payload those rows
would carry (for the checksum and the oracle), prints the record's fields as
one JSON line, and keeps the caches alive until a line arrives on stdin.

    python tests/ipc_exporter.py '{"layers": 28, "blocks": 96, ..., "imports": [[row, gen, block], ...]}'
"""
from __future__ import annotations

import json
import sys
from pathlib import Path
from types import SimpleNamespace

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def main() -> int:
    args = json.loads(sys.argv[1])
    import torch

    from cruise_amd.kv_transfer import capture_kv_device_transfer, release_kv_device_exports

    layers, blocks, bs, kvh, hd, batch = (args[k] for k in ("layers", "blocks", "block_size", "kv_heads", "head_dim", "batch"))
    gen = torch.Generator(device="cuda").manual_seed(args["seed"])
    # Every cache is allocated before any is filled, so each gets a fresh
    # allocation of its own size; the fill draws in place (no temporaries).
    caches = [tuple(torch.empty((blocks, bs, kvh, hd), dtype=torch.bfloat16, device="cuda") for _ in range(2))
              for _ in range(layers)]
    for pair in caches:
        for t in pair:
            t.normal_(0.0, 0.25, generator=gen)
    torch.cuda.synchronize()
    worker = SimpleNamespace(model_runner=SimpleNamespace(kv_caches=caches))
    requests = [SimpleNamespace(row=r, generation=g, scheduler_block_ids=(b,), kv_import_required=True)
                for r, g, b in args["imports"]]
    plan = SimpleNamespace(requests=requests, graph_batch_size=batch)
    transfer = capture_kv_device_transfer(worker, plan)

    # The payload the host path would carry: [K|V][layer][row][block].
    by_row = {r: b for r, _, b in args["imports"]}
    zero = torch.zeros((bs, kvh, hd), dtype=torch.bfloat16)
    parts = []
    for half in range(2):
        for layer in range(layers):
            for row in range(batch):
                block = by_row.get(row)
                parts.append(caches[layer][half][block].cpu() if block is not None else zero)
    Path(args["payload_path"]).write_bytes(torch.stack(parts).view(torch.uint16).numpy().tobytes())

    print(json.dumps({
        "transfer_id": transfer.transfer_id,
        "import_mask": transfer.import_mask,
        "row_generations": list(transfer.row_generations),
        "block_ids": list(transfer.block_ids),
        "source_bytes": transfer.source_bytes,
        "source_offsets": list(transfer.source_offsets),
        "keys": [k.hex() for k in transfer.keys],
        "allocations": len({int(t.data_ptr()) for pair in caches for t in pair}),
    }), flush=True)
    sys.stdin.readline()  # the importer is done with the caches
    release_kv_device_exports(worker)
    del caches
    torch.cuda.synchronize()
    return 0


if __name__ == "__main__":
    sys.exit(main())
