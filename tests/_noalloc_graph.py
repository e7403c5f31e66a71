"""Run in a fresh process by tests/test_zz_no_alloc.py: the first call of
tf_flash_decode_noalloc in the process is made under HIP stream capture
(torch.cuda.graph), so its per-device set-up runs during the capture.  The
graph is replayed twice, with eager work and synchronizations between the
replays, and each replay's output and Q8 must equal tf_flash_decode's with
a caller workspace bit for bit.  Prints "noalloc-graph ok" on success."""
import sys
from pathlib import Path

import numpy as np
import torch

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))
from taraference_amd import capi, synth  # noqa: E402


def main():
    lib = capi.load()
    rng = np.random.default_rng(91)
    n_head, n_kv, hd, L, n_split = 16, 2, 128, 1024, 16
    sc = float(np.float32(1 / np.sqrt(hd)))
    q = torch.from_numpy(rng.standard_normal(n_head * hd).astype(np.float32)).cuda()
    K = torch.from_numpy(synth.kv_cache(rng, L, n_kv, hd)).cuda()
    V = torch.from_numpy(synth.kv_cache(rng, L, n_kv, hd)).cuda()
    n = n_head * hd
    out_ref, q8_ref, d8_ref = (torch.empty(n, device="cuda"),
                               torch.empty(n, dtype=torch.int8, device="cuda"),
                               torch.empty(n // 32, device="cuda"))
    part = torch.empty(n_head * n_split * (2 + hd), device="cuda")
    rc = lib.tf_flash_decode(q.data_ptr(), K.data_ptr(), V.data_ptr(), part.data_ptr(), None,
                             out_ref.data_ptr(), q8_ref.data_ptr(), d8_ref.data_ptr(), n_head,
                             n_kv, hd, L - 1, None, n_split, sc, capi.stream_ptr())
    assert rc == 0, rc
    torch.cuda.synchronize()
    out, q8, d8 = torch.empty_like(out_ref), torch.empty_like(q8_ref), torch.empty_like(d8_ref)
    g = torch.cuda.CUDAGraph()
    print("[noalloc-graph] capturing the first call", flush=True)
    with torch.cuda.graph(g):
        rc = lib.tf_flash_decode_noalloc(q.data_ptr(), K.data_ptr(), V.data_ptr(),
                                         out.data_ptr(), q8.data_ptr(), d8.data_ptr(), n_head,
                                         n_kv, hd, L - 1, None, n_split, sc,
                                         capi.stream_ptr())
    assert rc == 0, rc
    for rep in range(2):
        out.fill_(float("nan"))
        q8.zero_()
        d8.zero_()
        torch.cuda.synchronize()
        print(f"[noalloc-graph] replay {rep}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), out_ref.view(torch.int32)), rep
        assert torch.equal(q8, q8_ref), rep
        assert torch.equal(d8.view(torch.int32), d8_ref.view(torch.int32)), rep
    print("noalloc-graph ok", flush=True)


if __name__ == "__main__":
    main()
