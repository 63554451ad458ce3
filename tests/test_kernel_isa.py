"""Static checks of the built gfx950 code objects (no GPU): the invariants the
kernels' correctness and occupancy rest on, read from their own assembly and
metadata (tests/kernel_isa.py).

- Every LDS tile is copied by buffer_load ... lds / global_load_lds, which the
  compiler does not track; the kernels rely on each wave waiting for its
  copies (vmcnt(0), or vmcnt(N) behind N later stores) before the workgroup
  barrier that publishes a tile.  Checked on every path of every kernel's
  control-flow graph.
- The register and LDS budgets that set the occupancy each kernel was
  designed for, and the absence of register spills where the design
  assumes none."""

import pytest

import kernel_isa as K

pytestmark = pytest.mark.skipif(not (K.tools_present() and K.images()),
                                reason="ROCm LLVM tools or built code objects absent")


def _all_kernels():
    out = []
    for image in K.images():
        for name in K.metadata(image):
            out.append((image, name))
    return out


def test_the_checker_finds_a_barrier_reached_with_a_copy_in_flight():
    # straight line: copy, barrier (bad); copy, wait, barrier (good)
    bad = [(0, "buffer_load_dwordx4", "v0, s[0:3], 0 offen lds", None),
           (8, "s_barrier", "", None), (12, "s_endpgm", "", None)]
    assert K.barriers_with_copy_in_flight(bad) == [8]
    good = [(0, "global_load_lds_dwordx4", "v[0:1], off", None),
            (8, "s_waitcnt", "vmcnt(0)", None), (12, "s_barrier", "", None),
            (16, "s_endpgm", "", None)]
    assert K.barriers_with_copy_in_flight(good) == []
    # a loop whose back edge carries a copy issued after the wait to the
    # barrier at the top of the loop body
    loop = [(0, "s_barrier", "", None),
            (4, "buffer_load_dword", "v1, s[0:3], 0 offen lds", None),
            (12, "s_cbranch_scc1", "", 0),
            (16, "s_waitcnt", "vmcnt(0)", None), (20, "s_endpgm", "", None)]
    assert K.barriers_with_copy_in_flight(loop) == [0]
    # the same loop with the wait inside it
    fixed = [(0, "s_barrier", "", None),
             (4, "buffer_load_dword", "v1, s[0:3], 0 offen lds", None),
             (12, "s_waitcnt", "vmcnt(0)", None), (16, "s_cbranch_scc1", "", 0),
             (20, "s_endpgm", "", None)]
    assert K.barriers_with_copy_in_flight(fixed) == []
    # a wait that leaves the N newest vector memory instructions in flight
    # covers a copy only if N stores follow it
    stores = [(0, "buffer_load_dword", "v1, s[0:3], 0 offen lds", None),
              (8, "global_store_dwordx4", "v[0:1], v[2:5], off", None),
              (16, "global_store_dwordx4", "v[0:1], v[2:5], off", None),
              (24, "s_waitcnt", "vmcnt(2)", None), (28, "s_barrier", "", None),
              (32, "s_endpgm", "", None)]
    assert K.barriers_with_copy_in_flight(stores) == []
    one_store = [stores[0], stores[1], stores[3], stores[4], stores[5]]
    assert K.barriers_with_copy_in_flight(one_store) == [28]
    # three buffers: copy A, barrier, copy B, wait leaving B in flight,
    # barrier (A landed: fine at depth 1), then a barrier with B still out
    ring = [(0, "buffer_load_dword", "v1, s[0:3], 0 offen lds", None),
            (8, "s_barrier", "", None),
            (12, "buffer_load_dword", "v1, s[0:3], 0 offen lds", None),
            (20, "s_waitcnt", "vmcnt(1)", None), (24, "s_barrier", "", None),
            (28, "s_barrier", "", None), (32, "s_endpgm", "", None)]
    assert K.barriers_with_copy_in_flight(ring, depth=1) == [28]
    assert K.barriers_with_copy_in_flight(ring, depth=0) == [8, 24]


def test_every_barrier_waits_for_the_waves_own_lds_copies():
    checked = 0
    for image in K.images():
        for name, insns in K.disassembly(image).items():
            if not any(K.is_lds_dma(mn, ops) for _, mn, ops, _ in insns):
                continue
            checked += 1
            # the 4-wave GEMM issues half of its second tile's copies before
            # its first barrier (they land by the second, before any wave
            # reads that tile): one barrier in flight
            depth = 1 if name.startswith(("tm_gemm_w4_", "tm_sae_w4_")) else 0
            bad = K.barriers_with_copy_in_flight(insns, depth)
            assert not bad, f"{name}: s_barrier at {[hex(a) for a in bad]} with an LDS copy in flight"
    assert checked >= 40  # the specialised attention and GEMM kernels


def _meta(prefix):
    out = {}
    for image in K.images():
        for name, m in K.metadata(image).items():
            if name.startswith(prefix):
                out[name] = m
    assert out, prefix
    return out


def test_forward_fits_two_waves_per_simd_without_spills():
    # (.vgpr_count is the unified count, VGPRs and AGPRs)
    # 256 registers per lane and at most half the CU's LDS per
    # workgroup: two workgroups of 4 waves per CU
    for name, m in _meta("tm_attn_fwd_fast_").items():
        assert m[".vgpr_count"] <= 256, name
        assert m[".vgpr_spill_count"] == 0 and m[".private_segment_fixed_size"] == 0, name
        assert m[".group_segment_fixed_size"] <= 80 * 1024, name


def test_dkdv_holds_its_accumulators_without_spills():
    for name, m in _meta("tm_attn_dkdv_fast_").items():
        assert m[".vgpr_spill_count"] == 0 and m[".private_segment_fixed_size"] == 0, name
        assert m[".vgpr_count"] <= 512, name
        if "_d128" in name:
            # head_dim 128 is the two-waves-per-SIMD build: 256 registers per
            # lane and at most half the CU's LDS (V rows plus two Q/dO buffers)
            assert m[".vgpr_count"] <= 256, name
            assert m[".group_segment_fixed_size"] <= 80 * 1024, name


def test_dq_fits_two_waves_per_simd_without_spills():
    for name, m in _meta("tm_attn_dq_fast_").items():
        assert m[".vgpr_count"] <= 256, name
        assert m[".vgpr_spill_count"] == 0 and m[".private_segment_fixed_size"] == 0, name
        assert m[".group_segment_fixed_size"] <= 80 * 1024, name


def test_gemm_and_sae_kernels_do_not_spill():
    for prefix in ("tm_gemm_fast_", "tm_gemm_ragged_", "tm_sae_fast_", "tm_sae_ragged_"):
        for name, m in _meta(prefix).items():
            assert m[".vgpr_spill_count"] == 0 and m[".private_segment_fixed_size"] == 0, name
            assert m[".group_segment_fixed_size"] <= 160 * 1024, name
