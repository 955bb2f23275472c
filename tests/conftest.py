"""Shared test setup: markers, import paths and the reference tests' generators."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "llm-inference-webgpu_amd")
for p in (PKG, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def lcg(n, seed):
    """The reference tests' generator: s = s*1664525 + 1013904223 mod 2^32,
    v = s/0xffffffff*2 - 1, stored f32 (test/quantize.test.js:10-18,
    test/attention.test.js:60-69, web/kernels.html:41-49)."""
    out = np.empty(n, np.float32)
    s = seed & 0xFFFFFFFF
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = (s / 0xFFFFFFFF) * 2 - 1
    return out


def lcg_fast(n, seed):
    """lcg() for large n: the same recurrence, vectorised by jumping ahead."""
    if n <= 4096:
        return lcg(n, seed)
    a, c, m = 1664525, 1013904223, 1 << 32
    block = 4096
    head = np.empty(block, np.uint64)
    s = seed & 0xFFFFFFFF
    for i in range(block):
        s = (s * a + c) % m
        head[i] = s
    # A^block, C_block for jumping `block` steps at once.
    A, C = 1, 0
    for _ in range(block):
        A, C = (A * a) % m, (C * a + c) % m
    out = np.empty(n, np.uint64)
    cur = head.copy()
    for start in range(0, n, block):
        k = min(block, n - start)
        out[start:start + k] = cur[:k]
        cur = (cur * np.uint64(A) + np.uint64(C)) % np.uint64(m)
    return ((out.astype(np.float64) / 0xFFFFFFFF) * 2 - 1).astype(np.float32)


@pytest.fixture(scope="session")
def hip():
    import qwen_hip
    qwen_hip.load_library()
    return qwen_hip


@pytest.fixture(scope="session")
def ctx(hip):
    """A context on device 0. Fails loudly when no GPU or library is present."""
    c = hip.GpuContext.create(0)
    yield c
    c.close()
