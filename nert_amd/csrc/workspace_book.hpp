// Bookkeeping for grow-only device workspaces and the HIP graphs that may
// hold their addresses. Host-only (no HIP types), so it is tested on the CPU.
//
// A captured graph bakes the workspace address into its kernel arguments. If
// a later eager call grows the workspace, freeing the old buffer would leave
// every live graph writing to freed memory on its next replay. So while any
// graph exec is alive, a replaced buffer is retired rather than freed, and
// the retired buffers are freed once the last graph exec is destroyed.

#pragma once

#include <cstddef>
#include <cstdint>
#include <utility>
#include <vector>

namespace nert_hip {

class WorkspaceBook {
  public:
    // A buffer was replaced by a larger one: the buffers that may be freed now
    // (the old one when no graph exec is alive, else none).
    std::vector<void*> Replaced(void* old) {
        if (old == nullptr) {
            return {};
        }
        if (live_graphs_ > 0) {
            retired_.push_back(old);
            return {};
        }
        return {old};
    }

    void GraphCreated() { ++live_graphs_; }

    // A graph exec was destroyed: the retired buffers that may be freed now.
    std::vector<void*> GraphDestroyed() {
        if (live_graphs_ > 0) {
            --live_graphs_;
        }
        if (live_graphs_ == 0) {
            return std::exchange(retired_, {});
        }
        return {};
    }

    int64_t live_graphs() const { return live_graphs_; }
    std::size_t retired() const { return retired_.size(); }

  private:
    int64_t live_graphs_ = 0;
    std::vector<void*> retired_;
};

} // namespace nert_hip
