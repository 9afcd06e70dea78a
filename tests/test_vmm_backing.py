"""The grow-on-demand VMM page backing (ref src/cache/cuda_vmm.rs:6-234,
pool.rs:287-322) on the CPU: the host-check build instantiates the same
VmmBacking template the HIP build does, over a mock of the VMM driver calls
that counts live reservations, physical handles and mappings and counts a
violation for every call that breaks a documented precondition of the VMM
API: sizes, addresses and alignments not multiples of the granularity (the
mock's is 64 KiB and an alignment-0 reservation comes back aligned to that
only), a mapping outside one live reservation, overlapping another, or of a
handle that is not live or already mapped, access set outside one live
mapping, an unmap that does not name exactly one mapping, a handle released
while mapped or twice, a reservation freed with another size or with
mappings inside.  One failure can be injected per run (reserve, create, map
or set_access at its n-th call).  The pool makes one reservation (alignment
0, as the reference) carved into its 2 L regions.

Checked: repeated create / grow / destroy cycles release everything; a
superblock that fails partway through its regions is rolled back (no region
keeps a mapping at that superblock, the superblock count does not advance,
the failed allocation leaves the pool unchanged), and the next growth maps it
again; ids and offsets stay equal to the oracle allocator's throughout.

The product library refuses KCMM_BACKING=vmm (see test_gpu_vmm.py)."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from lattice_amd.bindings import KV_BF16, make_config

RESERVE, CREATE, MAP, SET_ACCESS = 0, 1, 2, 3


@pytest.fixture
def vmm(hostcheck_lib, monkeypatch):
    monkeypatch.setenv("KCMM_BACKING", "vmm")
    lib = hostcheck_lib.lib
    lib.kcmm_hostcheck_vmm_reset.argtypes = [C.c_int, C.c_int64]
    lib.kcmm_hostcheck_vmm_state.argtypes = [C.POINTER(C.c_int64)]

    def state():
        out = (C.c_int64 * 4)()
        lib.kcmm_hostcheck_vmm_state(out)
        return dict(reservations=out[0], handles=out[1], mappings=out[2], violations=out[3])

    def arm(op=-1, at=-1):
        lib.kcmm_hostcheck_vmm_reset(op, at)

    arm()
    yield hostcheck_lib, state, arm
    arm()


CFG = dict(num_layers=3, kv_heads=8, head_dim=128, max_batch=4, max_seq_len=4096)   # 6 regions, 64 blocks per superblock


def test_cycles_release_everything(vmm):
    lib, state, arm = vmm
    base = state()
    for cycle in range(40):
        pool = lib.create_pool(make_config(**CFG), KV_BF16)
        assert pool.backing_kind() == 0
        n = 1 + 37 * (cycle % 5)                   # 1 .. 149 blocks: 1 .. 3 superblocks
        pool.alloc_blocks(n)
        sb = pool.stats()["superblock_count"]
        st = state()
        assert st["mappings"] - base["mappings"] == 6 * sb
        assert st["handles"] - base["handles"] == 6 * sb
        pool.destroy()
    assert state() == base and base["violations"] == 0


@pytest.mark.parametrize("op,region", [(SET_ACCESS, 3), (MAP, 4), (CREATE, 2), (SET_ACCESS, 0),
                                       (MAP, 5)])
def test_partial_superblock_rolls_back(vmm, op, region):
    """The second superblock fails at region `region` of 6: the mappings it
    made are undone, the allocation that needed it fails with nothing
    allocated, and a later allocation maps it and continues with the oracle's
    ids and offsets."""
    lib, state, arm = vmm
    pool = lib.create_pool(make_config(**CFG), KV_BF16)
    opool = O.OraclePool(16, 3, 8, 128, 4, 4096, O.BF16)
    try:
        bps = pool.stats()["blocks_per_superblock"]
        assert pool.alloc_blocks(bps) == opool.alloc(bps)           # superblock 0
        before = pool.stats()
        st0 = state()
        arm(op, region + 1)          # the (region+1)-th such call after arming fails
        with pytest.raises(Exception):
            pool.alloc_blocks(3)
        assert "mock" in pool.last_error()
        st1 = state()
        assert st1["mappings"] == st0["mappings"] and st1["handles"] == st0["handles"]
        assert st1["violations"] == 0
        assert pool.stats() == before
        arm()
        ids = pool.alloc_blocks(bps + 5)                             # superblocks 1 and 2
        assert ids == opool.alloc(bps + 5)
        assert np.array_equal(pool.all_block_offsets_f16(), opool.offsets_f16()[:pool.total_blocks()])
        assert pool.stats()["superblock_count"] == 3
        assert state()["mappings"] == 6 * 3 and state()["violations"] == 0
    finally:
        pool.destroy()
    assert state()["mappings"] == 0 and state()["handles"] == 0
    assert state()["reservations"] == 0 and state()["violations"] == 0


def test_failed_reservation_fails_creation_cleanly(vmm):
    lib, state, arm = vmm
    arm(RESERVE, 1)                                   # the pool's one reservation
    with pytest.raises(Exception):
        lib.create_pool(make_config(**CFG), KV_BF16)
    assert state() == dict(reservations=0, handles=0, mappings=0, violations=0)
