// CPU check of nert_amd/csrc/workspace_book.hpp: a workspace replaced while a
// captured graph exec is alive must not be freed until the last graph exec
// is destroyed. Prints "ok" and exits 0, or names the failed check and
// exits 1. Run by tests/test_runtime_host.py.

#include "../../nert_amd/csrc/workspace_book.hpp"

#include <cstdio>
#include <vector>

namespace {

int g_failures = 0;

void Expect(bool ok, const char* what) {
    if (!ok) {
        std::printf("FAILED: %s\n", what);
        ++g_failures;
    }
}

} // namespace

int main() {
    int a = 0, b = 0, c = 0, d = 0;
    nert_hip::WorkspaceBook book;
    // No graph alive: a replaced buffer is freed at once; null is ignored.
    Expect(book.Replaced(nullptr).empty(), "replacing null frees nothing");
    std::vector<void*> now = book.Replaced(&a);
    Expect(now.size() == 1 && now[0] == &a, "no graph: the old buffer is freed at once");
    // One graph alive: replacements are retired, not freed.
    book.GraphCreated();
    Expect(book.Replaced(&b).empty() && book.retired() == 1, "graph alive: the old buffer is retired");
    // A second graph, a second replacement; destroying one graph frees nothing.
    book.GraphCreated();
    Expect(book.Replaced(&c).empty() && book.retired() == 2, "two graphs: both replacements retired");
    Expect(book.GraphDestroyed().empty() && book.live_graphs() == 1, "one graph still alive: nothing freed");
    // The last graph goes: every retired buffer is handed back, once.
    now = book.GraphDestroyed();
    Expect(now.size() == 2 && now[0] == &b && now[1] == &c, "last graph destroyed: retired buffers freed");
    Expect(book.retired() == 0 && book.live_graphs() == 0, "book empty afterwards");
    Expect(book.GraphDestroyed().empty() && book.live_graphs() == 0, "extra destroy is harmless");
    // Back to no graphs: immediate frees again.
    now = book.Replaced(&d);
    Expect(now.size() == 1 && now[0] == &d, "no graph again: freed at once");
    if (g_failures == 0) {
        std::printf("ok\n");
    }
    return g_failures == 0 ? 0 : 1;
}
