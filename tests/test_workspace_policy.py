"""The workspace policy (ironmlx_amd/csrc/workspace_core.h) compiled for the
host with g++: requests reuse a grow-only buffer, grow outside capture, and
during capture never allocate -- a request the buffer cannot hold is refused,
so a captured graph holds kernel nodes only.  The call sequences are those of
the graph-capture tests: eager warm-up on one stream, capture on another."""
import os
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

DRIVER = r"""
#include <cstdio>
#include <map>
#include <utility>
#include "workspace_core.h"
using namespace iqmm;
// a simulated table of (stream, slot) -> capacity, counting allocations
struct Sim {
  std::map<std::pair<int,int>, size_t> cap;
  int allocs = 0, refused = 0;
  bool get(int st, int slot, size_t bytes, bool capturing) {
    size_t& c = cap[{st, slot}];
    switch (ws_decide(c, bytes, capturing)) {
      case WsDecision::Reuse: return true;
      case WsDecision::Grow: c = ws_grown_cap(c, bytes); ++allocs; return true;
      case WsDecision::CaptureTooSmall: ++refused; return false;
    }
    return false;
  }
};
int main() {
  // split-K partials (M=128, N=1024, ks=4), GLU product (M=40, 2I=3072, bf16),
  // offsets (E=64), sort histogram (65 buckets x 3 blocks)
  const size_t req[4] = {size_t(128) * 1024 * 4 * 4, size_t(40) * 3072 * 2, 65 * 8, 65 * 3 * 4};
  Sim s;
  for (int slot = 0; slot < 4; ++slot) if (!s.get(0, slot, req[slot], false)) return 1;
  const int eager_allocs = s.allocs;
  // capture on a fresh stream: every request refused, nothing allocated
  for (int slot = 0; slot < 4; ++slot) if (s.get(1, slot, req[slot], true)) return 2;
  if (s.allocs != eager_allocs || s.refused != 4) return 3;
  // capture on the warmed stream: reused, nothing allocated
  for (int slot = 0; slot < 4; ++slot) if (!s.get(0, slot, req[slot], true)) return 4;
  if (s.allocs != eager_allocs) return 5;
  // reservation (every slot to 4 MiB) on stream 1, then capture there
  for (int slot = 0; slot < 4; ++slot) s.get(1, slot, size_t(4) << 20, false);
  for (int slot = 0; slot < 4; ++slot) if (!s.get(1, slot, req[slot], true)) return 6;
  // growth: 1 MiB minimum, powers of two, never shrinks
  if (ws_grown_cap(0, 1) != (size_t(1) << 20)) return 7;
  if (ws_grown_cap(size_t(1) << 20, (size_t(3) << 20) + 1) != (size_t(4) << 20)) return 8;
  if (ws_decide(size_t(8) << 20, size_t(1) << 20, false) != WsDecision::Reuse) return 9;
  if (ws_decide(0, 0, true) != WsDecision::CaptureTooSmall) return 10;
  std::puts("ok");
  return 0;
}
"""


def test_workspace_policy_never_allocates_in_capture():
    with tempfile.TemporaryDirectory() as d:
        src = os.path.join(d, "drv.cpp")
        exe = os.path.join(d, "drv")
        with open(src, "w") as f:
            f.write(DRIVER)
        cc = subprocess.run(["g++", "-std=c++17", "-O1", "-fsanitize=address,undefined",
                             "-I", os.path.join(ROOT, "ironmlx_amd", "csrc"), src, "-o", exe],
                            capture_output=True, text=True)
        if cc.returncode != 0 and "sanitize" in cc.stderr:
            cc = subprocess.run(["g++", "-std=c++17", "-O1", "-I",
                                 os.path.join(ROOT, "ironmlx_amd", "csrc"), src, "-o", exe],
                                capture_output=True, text=True)
        assert cc.returncode == 0, cc.stderr
        r = subprocess.run([exe], capture_output=True, text=True)
        assert r.returncode == 0 and r.stdout.strip() == "ok", (r.returncode, r.stdout, r.stderr)


def test_workspace_sources_have_no_capture_allocation():
    """No caller frees (or owns) a per-call workspace any more: the only
    allocation is the grow path of workspace.hip."""
    csrc = os.path.join(ROOT, "ironmlx_amd", "csrc")
    for name in os.listdir(csrc):
        if not name.endswith((".hip", ".h")):
            continue
        with open(os.path.join(csrc, name)) as f:
            text = f.read()
        assert "hipFreeAsync" not in text, name
        assert text.count("hipMallocAsync(") == (1 if name == "workspace.hip" else 0), name
