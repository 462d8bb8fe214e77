"""The plugin products' workspace policy (joule_amd/csrc/jm_plugin_ws.h),
compiled on the host with g++ and checked case by case:

* under stream capture a call never takes the persistent buffer, even one
  large enough (a captured graph must not point at a buffer a later eager
  call may replace);
* otherwise a large-enough buffer is reused and a small one grown;
* growth at least doubles, so a stream's retired buffers (kept until the
  process ends) sum to less than its current one.
"""

import shutil
import subprocess
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parent.parent / "joule_amd" / "csrc"

DRIVER = r"""
#include <cstdio>
#include "jm_plugin_ws.h"
using jm::WsAction;
static int fails = 0;
#define CHECK(c) do { if (!(c)) { std::printf("FAIL line %d: %s\n", __LINE__, #c); fails++; } } while (0)
int main() {
    CHECK(jm::plugin_ws_action(1 << 20, 4096, true) == WsAction::StreamOrdered);
    CHECK(jm::plugin_ws_action(0, 4096, true) == WsAction::StreamOrdered);
    CHECK(jm::plugin_ws_action(1 << 20, 4096, false) == WsAction::Reuse);
    CHECK(jm::plugin_ws_action(4096, 4096, false) == WsAction::Reuse);
    CHECK(jm::plugin_ws_action(4095, 4096, false) == WsAction::Grow);
    CHECK(jm::plugin_ws_action(0, 1, false) == WsAction::Grow);
    CHECK(jm::plugin_ws_grow(0, 100) == ((size_t)1 << 20));
    CHECK(jm::plugin_ws_grow((size_t)1 << 20, (size_t)3 << 20) == ((size_t)3 << 20));
    CHECK(jm::plugin_ws_grow((size_t)4 << 20, (size_t)5 << 20) == ((size_t)8 << 20));
    // a stream that keeps asking for a little more: retired < current throughout
    size_t cur = 0, retired = 0;
    for (size_t need = 1000; need < ((size_t)1 << 34); need = need * 3 / 2 + 7) {
        if (jm::plugin_ws_action(cur, need, false) == WsAction::Grow) {
            retired += cur;
            cur = jm::plugin_ws_grow(cur, need);
            CHECK(cur >= need);
            CHECK(retired < cur);
        }
    }
    std::printf("%d failures\n", fails);
    return fails != 0;
}
"""


def test_plugin_ws_policy(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    src = tmp_path / "ws_policy.cpp"
    src.write_text(DRIVER)
    exe = tmp_path / "ws_policy"
    subprocess.run([gxx, "-std=c++17", "-O1", "-Wall", "-Werror", f"-I{CSRC}", str(src), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failures" in r.stdout
