// workspace.hip — device workspaces of the calls that need scratch memory
// (split-K partial sums, the gate_up product of a generic fused SwiGLU, the
// expert segment offsets of a grouped gather, the bucket counts of the MoE
// sort).
//
// Each (device, stream, slot) keeps one grow-only buffer, taken from the
// stream-ordered pool (hipMallocAsync on that stream, so it is ordered after
// the stream's earlier work) and never freed: HIP graphs captured on the
// stream keep pointing at it, so they hold kernel nodes only.  Calls on one
// stream execute in order, so they can share its buffers; a graph captured on
// a stream uses that stream's buffers and must not be replayed concurrently
// with other library work on that stream, or with another graph captured on
// it.  Nothing is allocated during capture (policy in workspace_core.h): a
// request that the buffer cannot hold then fails with
// hipErrorStreamCaptureUnsupported, and the caller sizes the buffers first
// (an eager call of the same shapes on the stream, or workspace_reserve).
#include <mutex>
#include <unordered_map>

#include "launch.h"
#include "workspace_core.h"

namespace iqmm {
namespace {

struct Key {
  int dev;
  hipStream_t st;
  int slot;
  bool operator==(const Key& o) const { return dev == o.dev && st == o.st && slot == o.slot; }
};
struct KeyHash {
  size_t operator()(const Key& k) const {
    return std::hash<const void*>()(static_cast<const void*>(k.st)) ^ (static_cast<size_t>(k.dev) << 48) ^
           (static_cast<size_t>(k.slot) << 56);
  }
};
struct Buf {
  void* p = nullptr;
  size_t cap = 0;
};

std::mutex g_mu;
std::unordered_map<Key, Buf, KeyHash>& table() {
  static auto* t = new std::unordered_map<Key, Buf, KeyHash>();  // lives until the process ends
  return *t;
}

}  // namespace

hipError_t workspace_get(hipStream_t st, int slot, size_t bytes, void** p) {
  *p = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(st, &cs);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lk(g_mu);
  Buf& b = table()[Key{dev, st, slot}];
  switch (ws_decide(b.cap, bytes, cs != hipStreamCaptureStatusNone)) {
    case WsDecision::Reuse:
      *p = b.p;
      return hipSuccess;
    case WsDecision::CaptureTooSmall:
      return hipErrorStreamCaptureUnsupported;
    case WsDecision::Grow: {
      // the old buffer stays allocated: graphs captured earlier point at it
      const size_t cap = ws_grown_cap(b.cap, bytes);
      void* np = nullptr;
      e = hipMallocAsync(&np, cap, st);
      if (e != hipSuccess) return e;
      b.p = np;
      b.cap = cap;
      *p = np;
      return hipSuccess;
    }
  }
  return hipErrorUnknown;
}

hipError_t workspace_reserve(hipStream_t st, size_t bytes) {
  for (int slot = 0; slot < WS_NSLOTS; ++slot) {
    void* p = nullptr;
    const hipError_t e = workspace_get(st, slot, bytes, &p);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace iqmm
