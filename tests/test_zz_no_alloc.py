"""The allocation-free flash decode (tf_flash_decode_noalloc, workspace in
the library's static device array) against tf_flash_decode with caller
workspace: two calls in a row, the second smaller, then a third at a long
context; outputs and Q8 bit-identical (the same kernels on the same
inputs), oversize requests rejected, and, in a fresh process, the first
call captured into a HIP graph and replayed."""
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from taraference_amd import synth
from _gpu import P, S, call, dev, empty, host

pytestmark = pytest.mark.gpu


def _pair(rng, n_head, n_kv, L, n_split):
    hd = 128
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    K, V = synth.kv_cache(rng, L, n_kv, hd), synth.kv_cache(rng, L, n_kv, hd)
    sc = float(np.float32(1 / np.sqrt(hd)))
    res = []
    for noalloc in (False, True):
        out, q8, d8 = empty(n_head * hd), empty(n_head * hd, torch.int8), empty(n_head * hd // 32)
        if noalloc:
            call("tf_flash_decode_noalloc", P(dev(q)), P(dev(K)), P(dev(V)), P(out), P(q8), P(d8),
                 n_head, n_kv, hd, L - 1, None, n_split, sc, S())
        else:
            part = empty(n_head * n_split * (2 + hd))
            cnt = torch.zeros(n_kv, dtype=torch.int32, device="cuda")
            call("tf_flash_decode", P(dev(q)), P(dev(K)), P(dev(V)), P(part), P(cnt), P(out),
                 P(q8), P(d8), n_head, n_kv, hd, L - 1, None, n_split, sc, S())
        res.append((host(out), host(q8), host(d8)))
    for a, b in zip(*res):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))


def test_noalloc_matches_workspace_entry(gpu):
    rng = np.random.default_rng(55)
    print("[no-alloc] 28/4 heads, L 4096, 64 splits", flush=True)
    _pair(rng, 28, 4, 4096, 64)
    print("[no-alloc] 16/2 heads, L 512, 8 splits (smaller)", flush=True)
    _pair(rng, 16, 2, 512, 8)
    print("[no-alloc] 16/2 heads, L 32768, 256 splits", flush=True)
    _pair(rng, 16, 2, 32768, 256)


def test_noalloc_rejects_oversize(gpu):
    from taraference_amd import capi

    out = empty(64 * 128)
    z = empty(16)
    # 64 heads x 256 splits x 130 floats > 2^20
    rc = capi.load().tf_flash_decode_noalloc(P(z), P(z), P(z), P(out), None, None, 64, 8, 128, 10,
                                            None, 256, 0.1, S())
    assert rc == 1  # hipErrorInvalidValue


def test_noalloc_first_call_under_graph_capture(gpu):
    """A fresh process (an empty per-device address cache) whose first call
    is captured: the set-up enqueues nothing into the graph."""
    script = Path(__file__).resolve().parent / "_noalloc_graph.py"
    print("[no-alloc] graph capture in a child process", flush=True)
    r = subprocess.run([sys.executable, str(script)], capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0 and "noalloc-graph ok" in r.stdout
