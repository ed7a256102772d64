"""The records the extraction keeps on the tensors it returns (event index on
time_steps, longest channel on cu_seqlens): they are read only while every
tensor they depend on is unchanged. CPU tensors stand in for device ones;
nothing here calls the library."""
import torch

from bc_mamba_amd import _provenance as prov


def _streams():
    t = torch.tensor([1, 4, 0, 2], dtype=torch.int32)
    ch = torch.tensor([0, 0, 1, 1], dtype=torch.int32)
    cu = torch.tensor([0, 2, 4], dtype=torch.int32)
    bm = torch.zeros((2, 32), dtype=torch.int32)
    ts = torch.zeros((2, 2), dtype=torch.int32)
    prov.attach_event_index(t, ch, cu, 8, bm, ts)
    return t, ch, cu, bm, ts


def test_index_found_for_its_own_tensors():
    t, ch, cu, bm, ts = _streams()
    got = prov.event_index_for(t, cu, 8)
    assert got is not None and got[0] is bm and got[1] is ts
    assert prov.event_index_for(t, None, 8, ch) is not None
    assert prov.event_index_for(t, cu.contiguous(), 8) is not None  # contiguous() of a contiguous tensor is itself


def test_index_ignored_after_any_change():
    t, ch, cu, bm, ts = _streams()
    assert prov.event_index_for(t, cu, 9) is None  # another seqlen
    assert prov.event_index_for(t.clone(), cu, 8) is None  # a copy carries no record
    assert prov.event_index_for(t, cu.clone(), 8) is None  # other offsets
    assert prov.event_index_for(t, None, 8, ch.clone()) is None  # other channel ids
    t2, ch2, cu2, _, _ = _streams()
    cu2[1] = 3  # offsets edited in place
    assert prov.event_index_for(t2, cu2, 8) is None
    t3, ch3, cu3, _, _ = _streams()
    ch3.add_(0)  # any in-place op bumps the version
    assert prov.event_index_for(t3, None, 8, ch3) is None and prov.event_index_for(t3, cu3, 8) is not None
    t4, _, cu4, bm4, _ = _streams()
    t4[0] = 2
    assert prov.event_index_for(t4, cu4, 8) is None
    t5, _, cu5, bm5, _ = _streams()
    bm5.zero_()  # the index itself edited
    assert prov.event_index_for(t5, cu5, 8) is None


def test_max_seqlen_record():
    cu = torch.tensor([0, 3, 5], dtype=torch.int32)
    assert prov.max_seqlen_of(cu) is None and not prov.covers_max_seqlen(cu, 10)
    prov.attach_max_seqlen(cu, 3)
    assert prov.max_seqlen_of(cu) == 3
    assert prov.covers_max_seqlen(cu, 3) and prov.covers_max_seqlen(cu, 4)
    assert not prov.covers_max_seqlen(cu, 2)  # an understated max_seqlen still gets the kernels' report
    assert prov.max_seqlen_of(cu.clone()) is None
    cu[2] = 9
    assert prov.max_seqlen_of(cu) is None and not prov.covers_max_seqlen(cu, 100)


def test_freed_dependency_voids_the_record():
    """A record keeps its channel_ids and cu_seqlens only weakly: once
    either is freed, nothing can match it (its memory may hold another
    tensor by then)."""
    import gc
    t, ch, cu, _, _ = _streams()
    assert prov.event_index_for(t, None, 8, ch) is not None
    del ch
    gc.collect()
    other = torch.zeros(4, dtype=torch.int32)  # may reuse the freed memory
    assert prov.event_index_for(t, None, 8, other) is None
    assert prov.event_index_for(t, cu, 8) is not None  # cu is still alive
    del cu
    gc.collect()
    assert prov.event_index_for(t, torch.tensor([0, 2, 4], dtype=torch.int32), 8) is None


def test_records_hold_no_reference_to_their_holder():
    import gc
    import weakref
    t, ch, cu, _, _ = _streams()
    prov.attach_max_seqlen(cu, 2)
    rt, rcu = weakref.ref(t), weakref.ref(cu)
    gc.disable()
    try:
        del t, cu
        # freed by reference counting alone: no record keeps a tensor alive
        # or forms a cycle
        assert rt() is None and rcu() is None
    finally:
        gc.enable()
