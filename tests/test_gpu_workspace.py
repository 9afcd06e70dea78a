"""Per-thread device scratch (split partials, attention partials) is freed
after its host thread exits: a server whose worker threads come and go must
not accumulate one set of buffers per thread that ever ran.  Seven threads
run the Cfg2 attention one after another (each needs about 10 MB of
partials); device free memory afterwards is within one thread's buffers of
what it was after the first thread."""
import threading

import numpy as np
import pytest

from lattice_amd.bindings import KV_BF16
from lattice_amd.workload import build_decode_case

pytestmark = pytest.mark.gpu


def test_exited_threads_release_their_workspaces(gpu_lib):
    import torch
    rng = np.random.default_rng(4)
    ctx = rng.integers(512, 4097, size=64) + 1
    case = build_decode_case(gpu_lib, batch=64, num_q_heads=32, kv_heads=8, head_dim=128,
                             block_size=16, ctx_lens=ctx, dtype=KV_BF16, seed=4,
                             host_mirror=False)
    stream = torch.cuda.Stream()
    errors = []

    def worker():
        try:
            case.run_attention(stream_ptr=stream.cuda_stream)
            stream.synchronize()
        except Exception as e:          # noqa: BLE001 -- reported by the main thread
            errors.append(e)

    def run_thread():
        t = threading.Thread(target=worker)
        t.start()
        t.join()

    try:
        run_thread()
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        for _ in range(6):
            run_thread()
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        assert not errors, errors
        lost = free0 - free1
        print(f"device memory held after 6 more worker threads: {lost / 2**20:.1f} MiB",
              flush=True)
        assert lost < 16 * 2**20, lost
        assert torch.isfinite(case.dev["out"].float()).all()
    finally:
        case.pool.destroy()
