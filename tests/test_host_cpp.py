"""The C++ host side: cvattn::kv_cache (cosyvoice.cpp_amd/host), the mirror of cosyvoice_kv_cache
(src/cosyvoice-kv-cache.h:9-69, src/cosyvoice-kv-cache.cpp).

The checks themselves live in the C++ program tests/cpp/kv_cache_test.  It drives the class the way
src/cosyvoice-llm.cpp and src/cosyvoice-token2wav.cpp drive cosyvoice_kv_cache, and compares
against the oracle: the cache bytes bit-exact, the attention within the fp tolerance.  These tests
run it.  The CPU test covers the argument checks that need no device.  The GPU test covers
everything else: LLM prefill/decode/offload/load in both attention modes, and DiT streaming slots.
"""
import ctypes
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "kv_cache_test")
HOST_LIB = os.path.join(ROOT, "cosyvoice.cpp_amd", "libcvattn_host.so")

# Itanium-mangled names of the class's public methods (g++, x86-64).
METHODS = {
    "build_kv_cache": "_ZN6cvattn8kv_cache14build_kv_cacheEiiiijiiiiib",
    "update_cache": "_ZN6cvattn8kv_cache12update_cacheER13cvattn_tensorS2_RKS1_iP12ihipStream_t",
    "update_cache_rope": "_ZN6cvattn8kv_cache17update_cache_ropeER13cvattn_tensorS2_RKS1_iliiffP12ihipStream_t",
    "set_input_v_idxs": "_ZN6cvattn8kv_cache16set_input_v_idxsEPKijjP12ihipStream_t",
    "attention_forward": "_ZN6cvattn8kv_cache17attention_forwardERK13cvattn_tensorS3_S3_PS2_S3_P12ihipStream_t",
    "shift_kv_node_pos": "_ZN6cvattn8kv_cache17shift_kv_node_posEj",
    "bind_slot": "_ZN6cvattn8kv_cache9bind_slotEi",
    "slide_kv_slot": "_ZN6cvattn8kv_cache13slide_kv_slotEv",
    "offload_slot": "_ZN6cvattn8kv_cache12offload_slotEijP12ihipStream_t",
    "load_slot": "_ZN6cvattn8kv_cache9load_slotEiP12ihipStream_t",
    "get_offloaded_cache_size": "_ZNK6cvattn8kv_cache24get_offloaded_cache_sizeEv",
    "clear_offloaded_cache": "_ZN6cvattn8kv_cache21clear_offloaded_cacheEv",
}


def run(args, timeout):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built (build() builds it)")
    r = subprocess.run([BIN] + args, capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    print(r.stderr)
    return r


def test_host_library_exports_the_methods():
    lib = ctypes.CDLL(HOST_LIB)
    missing = [m for m, sym in METHODS.items() if not hasattr(lib, sym)]
    assert not missing, missing


def test_argument_checks_without_a_device():
    r = run(["--no-gpu"], 60)
    assert r.returncode == 0 and "ALL PASSED" in r.stdout


@pytest.mark.gpu
def test_kv_cache_class_against_the_oracle():
    r = run([], 110)
    assert r.returncode == 0 and "ALL PASSED" in r.stdout, r.stdout[-4000:]
    # every case ran: 3 LLM caches x 6 steps x 2 layers, 2 DiT caches x 6 ODE steps x 2 layers
    assert r.stdout.count("ok   llm") == 36 and r.stdout.count("ok   dit") == 24
