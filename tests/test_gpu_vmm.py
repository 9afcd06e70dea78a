"""HIP VMM page backing on the GPU.

The backing is switched off in libkcmm.so: one process that created and
destroyed about a dozen VMM pools saw hipMemSetAccess fail ("invalid
argument") and then a crash in pool teardown, and no cause in this
library's code has been found (the bookkeeping, including the rollback of a
superblock that fails partway, is tested on the CPU in test_vmm_backing.py).
Until a cause is shown and fixed, KCMM_BACKING=vmm makes pool creation fail,
and the growth/parity/cycle test below stays skipped: it must not run on the
GPU before then."""
import math

import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import KV_BF16, KcmmError, make_config

pytestmark = pytest.mark.gpu


def test_vmm_backing_is_refused(gpu_lib, monkeypatch):
    monkeypatch.setenv("KCMM_BACKING", "vmm")
    with pytest.raises(KcmmError) as e:
        gpu_lib.create_pool(make_config(num_layers=1, kv_heads=2, head_dim=64, max_batch=2,
                                        max_seq_len=64), KV_BF16)
    assert "disabled" in str(e.value)


@pytest.mark.skip(reason="HIP VMM backing disabled: unexplained hipMemSetAccess failures and a "
                         "teardown crash after repeated pool create/destroy; not to be run on "
                         "the GPU until a cause is shown and fixed")
def test_vmm_growth_attention_parity_and_cycles(gpu_lib, monkeypatch):
    import torch
    from lattice_amd.workload import build_decode_case
    monkeypatch.setenv("KCMM_BACKING", "vmm")
    for cycle in range(12):
        case = build_decode_case(gpu_lib, batch=6, num_q_heads=32, kv_heads=8, head_dim=128,
                                 block_size=16, ctx_lens=[1, 300, 1025, 17, 700, 64],
                                 dtype=KV_BF16, seed=cycle)
        try:
            assert case.pool.backing_kind() == 0
            case.run_attention(stream_ptr=torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            g = case.geometry
            got = O.decode(O.BF16, case.out_bits()).astype(np.float64)
            ref = O.attn_decode_f64(KV_BF16, case.q_bits, case.k_mirror[0], case.v_mirror[0],
                                    case.block_tables, case.seq_lens, case.offsets_f16, 32, 8,
                                    128, 16, g["row_bytes"], g["data_bytes"], 1 / math.sqrt(128))
            assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-2
        finally:
            case.pool.destroy()
