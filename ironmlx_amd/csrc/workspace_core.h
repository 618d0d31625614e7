// workspace_core.h — the host-only policy of the per-(device, stream, slot)
// workspaces, free of HIP so that it is also compiled and tested on the CPU.
//
// A request is served from the slot's grow-only buffer when it fits.  When it
// does not, the buffer grows (x2 steps, 1 MiB minimum) outside stream capture.
// During capture nothing is allocated: a graph must only hold kernel nodes
// that point at buffers that outlive it, so a request larger than the
// buffer fails (WsDecision::CaptureTooSmall) and the caller reports it; the
// stream's workspaces are sized beforehand by an eager call of the same
// shapes on that stream or by an explicit reservation.
#pragma once
#include <stddef.h>

namespace iqmm {

enum class WsDecision { Reuse, Grow, CaptureTooSmall };

constexpr size_t kWsMinCap = size_t{1} << 20;

// new capacity of a buffer of capacity `cap` that must hold `bytes`
inline size_t ws_grown_cap(size_t cap, size_t bytes) {
  size_t c = cap ? cap : kWsMinCap;
  while (c < bytes) c *= 2;
  return c;
}

inline WsDecision ws_decide(size_t cap, size_t bytes, bool capturing) {
  if (bytes == 0) bytes = 1;
  if (cap >= bytes) return WsDecision::Reuse;
  return capturing ? WsDecision::CaptureTooSmall : WsDecision::Grow;
}

}  // namespace iqmm
