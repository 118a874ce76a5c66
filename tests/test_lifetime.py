"""Handle lifetimes of the C ABI, on the CPU.

libgemma_hip's host code (model.cpp, gguf.cpp, repack.cpp, synth.cpp) is
built with g++ and AddressSanitizer against a host-only stand-in for the
HIP runtime (tests/cpp/hip_stub.cpp: streams, events and graphs are heap
objects each call dereferences) and no-op kernel launchers
(tests/cpp/kernel_stub.cpp), then driven by tests/cpp/lifetime_test.cpp:
every destroy order of context, model, cache and Q4_0 tensor must be free
of use-after-free and leaks (finalisers run in any order:
src/Gemma/KVCache.hs:20-35 handles under a -threaded RTS, gemma.cabal:102),
and a second destroy is GH_ERR_STATE.  A second driver mode runs a
stepping thread beside a destroying one (under AddressSanitizer and under
ThreadSanitizer) to show the lock order cannot deadlock.
"""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from conftest import REPO

CSRC = REPO / "gemma.hs_amd" / "csrc"
CPP = REPO / "tests" / "cpp"


def build_lifetime_test(out_dir, sources=None, sanitizer="address"):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    srcs = sources or [CSRC / f for f in ("model.cpp", "gguf.cpp", "repack.cpp", "synth.cpp")]
    exe = out_dir / "lifetime_test"
    cmd = [gxx, "-std=c++17", "-g", "-O1", f"-fsanitize={sanitizer}", "-fno-omit-frame-pointer",
           "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{REPO / 'include'}",
           *map(str, srcs), str(CPP / "hip_stub.cpp"), str(CPP / "kernel_stub.cpp"),
           str(CPP / "lifetime_test.cpp"), "-o", str(exe), "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    return exe


@pytest.fixture(scope="module")
def lifetime_exe(tmp_path_factory):
    return build_lifetime_test(tmp_path_factory.mktemp("lifetime"))


@pytest.fixture(scope="module")
def lifetime_tsan_exe(tmp_path_factory):
    return build_lifetime_test(tmp_path_factory.mktemp("lifetime_tsan"), sanitizer="thread")


def _run(exe, *args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=23",
               TSAN_OPTIONS="halt_on_error=1:exitcode=24")
    env.pop("LD_PRELOAD", None)
    return subprocess.run([str(exe), *args], capture_output=True, text=True, env=env, timeout=300)


def test_handles_destroyed_in_any_order_are_clean_under_asan(lifetime_exe):
    r = _run(lifetime_exe)
    assert r.returncode == 0 and "lifetime ok" in r.stdout, r.stdout + r.stderr[-4000:]


def test_destroy_during_a_step_on_another_thread_does_not_deadlock(lifetime_exe):
    """A finaliser thread destroying caches, Q4_0 tensors and models on a
    context while another thread steps, samples and rewinds on it: the
    registry mutex is never held while a context mutex is taken, so neither
    waits on the other (a watchdog exits 3 on a deadlock)."""
    r = _run(lifetime_exe, "race")
    assert r.returncode == 0 and "race ok" in r.stdout, r.stdout + r.stderr[-4000:]


def test_concurrent_step_and_destroy_are_free_of_data_races_under_tsan(lifetime_tsan_exe):
    """The same two threads under ThreadSanitizer: every host field a call
    reads or writes (cache lengths, children lists, released flags) is
    guarded by the context mutex."""
    r = _run(lifetime_tsan_exe, "race")
    assert r.returncode == 0 and "race ok" in r.stdout, r.stdout + r.stderr[-4000:]


def test_interpreter_exit_finaliser_order_is_clean_under_asan(lifetime_exe):
    """Context destroyed first, then the model, then its cache: the order
    that, before handles were reference counted, read the freed context."""
    r = _run(lifetime_exe, "exit")
    assert r.returncode == 0 and "exit order ok" in r.stdout, r.stdout + r.stderr[-4000:]


def test_model_create_rejects_unsupported_configs(lifetime_exe):
    """gh_model_create refuses, with GH_ERR_INVALID and no handle, the
    configurations the kernels do not support (hidden above 3072 or not a
    multiple of 32, head_dim other than 32/128/256, groups other than
    1/2/4/8) and malformed ones (negative window or global period, RoPE
    theta not finite and > 0, eps negative or NaN, unknown mode, no KV
    capacity); hidden 3072 is accepted."""
    r = _run(lifetime_exe, "config")
    assert r.returncode == 0 and "config ok" in r.stdout, r.stdout + r.stderr[-4000:]
