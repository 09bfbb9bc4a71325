"""CPU: host-side runtime bookkeeping that needs no GPU.

The workspace book (nert_amd/csrc/workspace_book.hpp) keeps a grown
workspace's old buffer alive while any captured HIP graph may still use its
address (tests/cpp/workspace_book_test.cpp)."""

import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_workspace_book():
    exe = ROOT / "tests" / "_build" / "workspace_book_test"
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0 and proc.stdout.strip() == "ok", proc.stdout + proc.stderr
