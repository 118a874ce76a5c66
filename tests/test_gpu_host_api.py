"""The C++ host API (gemma.hs_amd/host/Gemma.hpp) on the MI355X (marked gpu).

The reference's host side is Haskell; without GHC here, the API above the C
ABI is mirrored in C++ with the reference's names, argument meaning and
error behaviour.  tests/cpp/host_api_test.cpp exercises it against the C
oracle; this test runs those checks in-process (built by build() as
tests/cpp/libhost_api_test.so):
- runGemmaInferenceCached / runGemmaInferenceCachedWithLayer0 step by step:
  logits and layer 0 within 1e-4 of the oracle, sampleToken equal to the
  oracle's argmax, cacheLength growing by one, a fresh 2048-position cache
  when none is given (tiny config, f32 and Q4_0 weights);
- generate, token by token and with the batched prefill: the oracle's ids;
- two tokens: GemmaError "Cached inference requires single token, got 2"
  (src/Gemma/Model.hs:1321-1324), the cache unchanged; a full cache:
  GH_ERR_RANGE;
- runLinearQ4 on raw GGUF words, with and without soft-cap, against the
  oracle's Q4_0 matvec.
"""
from __future__ import annotations

import ctypes as C

import pytest

import gemma_hip as gh
from conftest import REPO

pytestmark = pytest.mark.gpu


def test_cpp_host_api_against_oracle():
    gh.lib()  # the in-tree libgemma_hip, which the test library links
    path = REPO / "tests" / "cpp" / "libhost_api_test.so"
    assert path.exists(), "build() builds tests/cpp/libhost_api_test.so"
    t = C.CDLL(str(path))
    t.gh_host_api_tests.restype = C.c_int
    t.gh_host_api_tests.argtypes = [C.c_char_p, C.c_int]
    buf = C.create_string_buffer(8192)
    rc = t.gh_host_api_tests(buf, len(buf))
    log = buf.value.decode()
    print(log)
    assert rc == 0, log
    for line in ("errors ok", "runLinearQ4 ok", "tiny f32:", "tiny q4:"):
        assert line in log, log
