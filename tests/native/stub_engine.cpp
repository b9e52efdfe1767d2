// Test double of the engine's C-ABI (resident_epoch_create / execute /
// destroy) for CPU tests of the sidecar server: the server binary is linked
// against this library instead of the HIP one, so every operation of the
// socket protocol can be driven without a GPU.
//
// Behaviour (fully determined by the inputs, so the tests can predict it):
// * create: fails with status STUB_CREATE_STATUS when that variable is set
//   and non-zero; appends its five path arguments to STUB_LOG.
// * execute: every row with a generation runs max_steps steps emitting
//   token + step + 1; the request count must equal the rows with a
//   generation (else 12).  Host-file import: the transfer file's header must
//   carry transfer_id (else 13); the reported checksum is the header's.
//   Device IPC: the reported checksum is 0x1000 + import_mask + 16 *
//   block_ids[first imported row]; a zero magic returns 35.  The transfer
//   path (or "-") is appended to STUB_LOG.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "resident_epoch.h"

namespace {

void log_line(const char* text) {
  const char* path = getenv("STUB_LOG");
  if (path == nullptr) return;
  FILE* f = fopen(path, "a");
  if (f == nullptr) return;
  fprintf(f, "%s\n", text);
  fclose(f);
}

int g_engine = 0;

}  // namespace

extern "C" void* resident_epoch_create(const char* air, const char* graph_config, const char* func_config,
                                       const char* weights, const char* tiling, int32_t* status) {
  const char* forced = getenv("STUB_CREATE_STATUS");
  const int s = forced != nullptr ? atoi(forced) : 0;
  char line[4096];
  snprintf(line, sizeof(line), "create %s %s %s %s %s", air, graph_config, func_config, weights, tiling);
  log_line(line);
  *status = s;
  return s == 0 ? &g_engine : nullptr;
}

extern "C" int32_t resident_epoch_execute(
    void* engine, int32_t request_count, int32_t max_steps, const int64_t* tokens, const int64_t* positions,
    const int32_t* lengths, const int32_t* eos, const int32_t* gens, int64_t* out_tokens, int32_t* out_executed,
    int32_t* out_gens, int32_t* model_calls, int32_t* device_status, int32_t* feed_calls, int32_t* fetch_calls,
    int32_t* commit_state, int32_t* checksum, int64_t* wall_us, int64_t* native_cpu_us, int64_t* in_bytes,
    int64_t* out_bytes, const char* transfer_path, uint64_t transfer_id, const ResidentEpochIpcMetadata* ipc) {
  (void)positions;
  (void)lengths;
  (void)eos;
  *commit_state = CRUISE_EPOCH_PREPARED;
  if (engine != &g_engine) return 10;
  char line[4096];
  snprintf(line, sizeof(line), "execute %s %llu", transfer_path ? transfer_path : "-",
           static_cast<unsigned long long>(transfer_id));
  log_line(line);
  int active = 0;
  for (int r = 0; r < 4; ++r) active += gens[r] != 0;
  if (active != request_count) return 12;
  uint32_t sum = 0;
  if (transfer_path != nullptr) {
    FILE* f = fopen(transfer_path, "rb");
    unsigned char header[CRUISE_RESIDENT_TRANSFER_HEADER_BYTES];
    const bool ok = f != nullptr && fread(header, 1, sizeof(header), f) == sizeof(header);
    if (f != nullptr) fclose(f);
    uint64_t id = 0;
    if (ok) memcpy(&id, header + 16, 8);
    if (!ok || id != transfer_id) return 13;
    memcpy(&sum, header + 76, 4);
  } else if (ipc != nullptr) {
    if (ipc->magic == 0) return 35;
    int first = 0;
    while (first < 4 && (ipc->import_mask & (1u << first)) == 0) ++first;
    sum = 0x1000u + ipc->import_mask + 16u * static_cast<uint32_t>(first < 4 ? ipc->block_ids[first] : 0);
  }
  *commit_state = CRUISE_EPOCH_EXECUTING;
  for (int i = 0; i < 32; ++i) out_tokens[i] = -1;
  for (int r = 0; r < 4; ++r) {
    out_gens[r] = gens[r];
    out_executed[r] = gens[r] != 0 ? max_steps : 0;
    for (int s = 0; s < out_executed[r]; ++s) out_tokens[r * 8 + s] = tokens[r] + s + 1;
  }
  *model_calls = max_steps;
  *device_status = 0;
  *feed_calls = 1;
  *fetch_calls = 1;
  *checksum = static_cast<int32_t>(sum);
  *wall_us = 5;
  *native_cpu_us = 3;
  *in_bytes = transfer_path != nullptr ? CRUISE_RESIDENT_IMPORT_INPUT_BYTES : 260;
  *out_bytes = 368;
  *commit_state = CRUISE_EPOCH_COMMITTED;
  return 0;
}

extern "C" void resident_epoch_destroy(void* engine) {
  (void)engine;
  log_line("destroy");
}

// Only "batch" is known: 4, or STUB_BATCH when set.
extern "C" int32_t resident_epoch_info(void* engine, const char* key, int64_t* value) {
  if (engine != &g_engine || key == nullptr || value == nullptr || strcmp(key, "batch") != 0) return -1;
  const char* forced = getenv("STUB_BATCH");
  *value = forced != nullptr ? atoi(forced) : 4;
  return 0;
}
