"""The allocator's out-of-memory policy (tensors_amd/csrc/alloc_policy.hpp,
used by tf_hip_alloc and the workspace growth) driven on the host with fake
allocators: a retry happens exactly once, only after an out-of-memory, and
only when releasing the held-back memory freed something."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]

DRIVER = r'''
#include "alloc_policy.hpp"
#include <cstdio>
#include <vector>
using tfh::AllocOutcome;
struct Fake {
    std::vector<AllocOutcome> script;  // outcome of each attempt, in order
    bool frees = true;                 // what release() reports
    int attempts = 0, releases = 0;
    AllocOutcome run() {
        return tfh::allocate_with_retry(
            [&] { return script[attempts++]; },
            [&] { ++releases; return frees; });
    }
};
#define EXPECT(c) do { if (!(c)) { std::printf("FAIL line %d: %s\n", __LINE__, #c); return 1; } } while (0)
int main() {
    { Fake f{{AllocOutcome::Ok}}; EXPECT(f.run() == AllocOutcome::Ok); EXPECT(f.attempts == 1 && f.releases == 0); }
    { Fake f{{AllocOutcome::OutOfMemory, AllocOutcome::Ok}};
      EXPECT(f.run() == AllocOutcome::Ok); EXPECT(f.attempts == 2 && f.releases == 1); }
    { Fake f{{AllocOutcome::OutOfMemory, AllocOutcome::OutOfMemory}};
      EXPECT(f.run() == AllocOutcome::OutOfMemory); EXPECT(f.attempts == 2 && f.releases == 1); }
    { Fake f{{AllocOutcome::OutOfMemory}, false};
      EXPECT(f.run() == AllocOutcome::OutOfMemory); EXPECT(f.attempts == 1 && f.releases == 1); }
    { Fake f{{AllocOutcome::Failed}}; EXPECT(f.run() == AllocOutcome::Failed); EXPECT(f.attempts == 1 && f.releases == 0); }
    { Fake f{{AllocOutcome::OutOfMemory, AllocOutcome::Failed}};
      EXPECT(f.run() == AllocOutcome::Failed); EXPECT(f.attempts == 2); }
    std::printf("OK\n");
    return 0;
}
'''


@pytest.mark.skipif(shutil.which("g++") is None, reason="no host C++ compiler")
def test_alloc_retry_policy(tmp_path):
    src = tmp_path / "drive.cpp"
    src.write_text(DRIVER)
    exe = tmp_path / "drive"
    subprocess.run(["g++", "-std=c++17", "-O1", f"-I{ROOT / 'tensors_amd' / 'csrc'}", str(src), "-o", str(exe)],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "OK", r.stdout + r.stderr
