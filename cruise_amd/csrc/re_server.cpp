// Sidecar server of the resident decode epoch: one engine per process, driven
// over a Unix stream socket by the Python sidecar client.
//
// Replaces native/resident_epoch_server.cpp (the reference's sidecar).  The
// command line, the wire records (136-byte request, 352-byte response,
// protocol version 7), the operation codes, the startup response and the exit
// statuses are the reference's, so its Python client (sidecar_backend.py:
// 23-35, 150-194) drives this server unchanged:
//
//   resident_epoch_server SOCKET AIR GRAPH_CONFIG FUNC_CONFIG WEIGHTS TILING
//
//   SOCKET must lie under /dev/shm/.  The server listens, accepts one client,
//   creates the engine (resident_epoch_create with the other five
//   arguments), sends a startup response whose transport status is 0 or
//   100 + the create status (101 also for an engine whose batch is not the
//   wire records' four rows), and then serves one request at a time:
//     1 EXECUTE, 2 WARM_UP      resident_epoch_execute, no KV import
//     4 IMPORT_EXECUTE          import from the host snapshot file
//                               SOCKET + ".kv-transfer" (deleted afterwards)
//     5 DEVICE_IPC_EXECUTE      the request is followed by the 4,088-byte
//                               device-IPC metadata record
//     3 SHUTDOWN                empty response, then exit 0
//   A request with the wrong magic or version gets transport status 69, an
//   unknown operation 71; both keep the connection.
//
// Exit statuses: 64 usage, 65 listener, 66 accept, 67 startup response not
// delivered, 68 client gone, 70 shutdown response not delivered, 72 response
// not delivered, 73 IPC metadata not received, 100 + s engine creation
// failed with status s.
#include <errno.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/socket.h>
#include <sys/un.h>
#include <unistd.h>

#include <string>

#include "resident_epoch.h"
#include "resident_epoch_protocol.h"

namespace {

constexpr uint32_t kRequestMagic = 0x71317131u;
constexpr uint32_t kResponseMagic = 0x71327132u;
constexpr int kRows = 4;       // rows of the wire record
constexpr int kMaxSteps = 8;   // history slots per row of the wire record

enum Operation : uint16_t {
  kExecute = 1,
  kWarmUp = 2,
  kShutdown = 3,
  kImportExecute = 4,
  kDeviceIpcExecute = 5,
};

enum ExitStatus : int {
  kExitOk = 0,
  kExitUsage = 64,
  kExitListener = 65,
  kExitAccept = 66,
  kExitStartupSend = 67,
  kExitClientGone = 68,
  kExitShutdownSend = 70,
  kExitResponseSend = 72,
  kExitIpcMetadata = 73,
  kExitCreateBase = 100,
};

constexpr int32_t kTransportBadHeader = 69;
constexpr int32_t kTransportBadOperation = 71;

// Little-endian packed records, field order of sidecar_backend.py:34-35
// (REQUEST "<IHHiiQ4q4q4i4i4i", RESPONSE "<Iiiiiiii4q4i4i32q").
#pragma pack(push, 1)
struct WireRequest {
  uint32_t magic;
  uint16_t version;
  uint16_t operation;
  int32_t request_count;
  int32_t max_steps;
  uint64_t transfer_id;
  int64_t token_ids[kRows];
  int64_t positions[kRows];
  int32_t sequence_lengths[kRows];
  int32_t eos_token_ids[kRows];
  int32_t row_generations[kRows];
};

struct WireResponse {
  uint32_t magic;
  int32_t transport_status;
  int32_t device_status;
  int32_t model_calls;
  int32_t feed_calls;
  int32_t fetch_calls;
  int32_t commit_state;
  int32_t kv_import_checksum;
  int64_t wall_us;
  int64_t native_cpu_us;
  int64_t declared_input_bytes;
  int64_t declared_output_bytes;
  int32_t executed[kRows];
  int32_t row_generations[kRows];
  int64_t token_ids[kRows * kMaxSteps];
};
#pragma pack(pop)

static_assert(sizeof(WireRequest) == CRUISE_SIDECAR_REQUEST_BYTES, "request record size");
static_assert(sizeof(WireResponse) == CRUISE_SIDECAR_RESPONSE_BYTES, "response record size");
static_assert(sizeof(ResidentEpochIpcMetadata) == CRUISE_RESIDENT_IPC_METADATA_BYTES, "IPC metadata size");

// Moves exactly n bytes; false on end of stream or an error other than EINTR.
bool recv_exact(int fd, void* dst, size_t n) {
  uint8_t* p = static_cast<uint8_t*>(dst);
  while (n > 0) {
    const ssize_t got = ::recv(fd, p, n, 0);
    if (got > 0) {
      p += got;
      n -= static_cast<size_t>(got);
    } else if (got == 0 || errno != EINTR) {
      return false;
    }
  }
  return true;
}

bool send_exact(int fd, const void* src, size_t n) {
  const uint8_t* p = static_cast<const uint8_t*>(src);
  while (n > 0) {
    // MSG_NOSIGNAL: a client that went away is an error status, not SIGPIPE.
    const ssize_t put = ::send(fd, p, n, MSG_NOSIGNAL);
    if (put >= 0) {
      p += put;
      n -= static_cast<size_t>(put);
    } else if (errno != EINTR) {
      return false;
    }
  }
  return true;
}

// The response every reply starts from: no device status yet, PREPARED, no
// rows executed, history filled with -1 (sidecar_backend.py reads tokens only
// up to each row's executed count).
WireResponse blank_response(int32_t transport_status) {
  WireResponse r;
  memset(&r, 0, sizeof(r));
  r.magic = kResponseMagic;
  r.transport_status = transport_status;
  r.device_status = -1;
  r.commit_state = CRUISE_EPOCH_PREPARED;
  for (int64_t& t : r.token_ids) t = -1;
  return r;
}

// A listening socket at path (must be under /dev/shm/, like every other file
// the engine exchanges); -1 on failure.
int listen_at(const std::string& path) {
  if (path.compare(0, 9, "/dev/shm/") != 0) return -1;
  sockaddr_un addr;
  memset(&addr, 0, sizeof(addr));
  if (path.size() >= sizeof(addr.sun_path)) return -1;
  addr.sun_family = AF_UNIX;
  memcpy(addr.sun_path, path.c_str(), path.size() + 1);
  const int fd = ::socket(AF_UNIX, SOCK_STREAM, 0);
  if (fd < 0) return -1;
  ::unlink(path.c_str());
  if (::bind(fd, reinterpret_cast<const sockaddr*>(&addr), sizeof(addr)) != 0 || ::listen(fd, 1) != 0) {
    ::close(fd);
    ::unlink(path.c_str());
    return -1;
  }
  return fd;
}

class Session {
 public:
  Session(std::string socket_path, int listener, int client)
      : socket_path_(std::move(socket_path)),
        transfer_path_(socket_path_ + ".kv-transfer"),
        listener_(listener),
        client_(client) {}

  ~Session() {
    if (engine_ != nullptr) resident_epoch_destroy(engine_);
    ::close(client_);
    ::close(listener_);
    ::unlink(socket_path_.c_str());
    ::unlink(transfer_path_.c_str());
  }

  // Creates the engine and reports the result to the client.
  int start(char** create_args) {
    int32_t status = -1;
    engine_ = resident_epoch_create(create_args[0], create_args[1], create_args[2], create_args[3], create_args[4],
                                    &status);
    // The wire records carry four rows: an engine of any other batch cannot
    // be served and is reported as a creation failure with bad arguments (1).
    int64_t batch = 0;
    if (engine_ != nullptr && (resident_epoch_info(engine_, "batch", &batch) != 0 || batch != kRows)) {
      resident_epoch_destroy(engine_);
      engine_ = nullptr;
      status = 1;
    }
    const int32_t transport = engine_ == nullptr ? kExitCreateBase + status : 0;
    const WireResponse startup = blank_response(transport);
    const bool sent = send_exact(client_, &startup, sizeof(startup));
    if (engine_ == nullptr) return transport;
    return sent ? kExitOk : kExitStartupSend;
  }

  // Serves requests until shutdown or a transport failure.
  int serve() {
    for (;;) {
      WireRequest req;
      if (!recv_exact(client_, &req, sizeof(req))) return kExitClientGone;
      WireResponse resp = blank_response(0);
      if (req.magic != kRequestMagic || req.version != CRUISE_SIDECAR_PROTOCOL_VERSION) {
        resp.transport_status = kTransportBadHeader;
      } else if (req.operation == kShutdown) {
        return send_exact(client_, &resp, sizeof(resp)) ? kExitOk : kExitShutdownSend;
      } else if (req.operation == kExecute || req.operation == kWarmUp || req.operation == kImportExecute ||
                 req.operation == kDeviceIpcExecute) {
        const int rc = run_epoch(req, resp);
        if (rc != kExitOk) return rc;
      } else {
        resp.transport_status = kTransportBadOperation;
      }
      if (!send_exact(client_, &resp, sizeof(resp))) return kExitResponseSend;
    }
  }

 private:
  int run_epoch(const WireRequest& req, WireResponse& resp) {
    ResidentEpochIpcMetadata ipc;
    const ResidentEpochIpcMetadata* ipc_arg = nullptr;
    if (req.operation == kDeviceIpcExecute) {
      if (!recv_exact(client_, &ipc, sizeof(ipc))) return kExitIpcMetadata;
      ipc_arg = &ipc;
    }
    const bool file_import = req.operation == kImportExecute;
    resp.transport_status = resident_epoch_execute(
        engine_, req.request_count, req.max_steps, req.token_ids, req.positions, req.sequence_lengths,
        req.eos_token_ids, req.row_generations, resp.token_ids, resp.executed, resp.row_generations,
        &resp.model_calls, &resp.device_status, &resp.feed_calls, &resp.fetch_calls, &resp.commit_state,
        &resp.kv_import_checksum, &resp.wall_us, &resp.native_cpu_us, &resp.declared_input_bytes,
        &resp.declared_output_bytes, file_import ? transfer_path_.c_str() : nullptr, req.transfer_id, ipc_arg);
    // The snapshot file is single use, whatever the outcome.
    if (file_import) ::unlink(transfer_path_.c_str());
    return kExitOk;
  }

  const std::string socket_path_;
  const std::string transfer_path_;
  const int listener_;
  const int client_;
  void* engine_ = nullptr;
};

}  // namespace

int main(int argc, char** argv) {
  if (argc != 7) {
    fprintf(stderr, "usage: %s SOCKET AIR GRAPH_CONFIG FUNC_CONFIG WEIGHTS TILING\n", argv[0]);
    return kExitUsage;
  }
  const std::string socket_path = argv[1];
  const int listener = listen_at(socket_path);
  if (listener < 0) return kExitListener;
  int client;
  do {
    client = ::accept(listener, nullptr, nullptr);
  } while (client < 0 && errno == EINTR);
  if (client < 0) {
    ::close(listener);
    ::unlink(socket_path.c_str());
    return kExitAccept;
  }
  Session session(socket_path, listener, client);
  const int started = session.start(argv + 2);
  if (started != kExitOk) return started;
  return session.serve();
}
