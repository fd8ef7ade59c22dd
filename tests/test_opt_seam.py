"""The Opt seam remapped onto template parameters (codegen/opt.go:29-72, beam.go:41-72), host only:
ApplyOpts edits a gemm key's tuning parameters, ActionSpace lists exactly the Opts that change the
kernel into another instantiated one, and invalid sequences fail closed."""
import pytest

from anneal_amd import _lib as L
from anneal_amd.executor import action_space, apply_opts

F16 = "tmpl:gemm;dtype=f16;epi=bias_relu;ta=0;tb=0;M=4096;N=4096;K=1024"
F32 = "tmpl:gemm;dtype=f32;epi=store;ta=1;tb=1;M=128;N=784;K=64"


def params(key):
    return dict(kv.split("=") for kv in key.split(";")[1:])


def test_local_upcast_tile_pick_instantiated_variants():
    # the shape's default is variant 3 (256x256, 4x2 waves); LOCAL(axis 0, 16) keeps the tile on 2x2 waves
    two_by_two = apply_opts(F16, [(L.OPT_LOCAL, 0, 16)])
    assert params(two_by_two)["variant"] == "2"          # 256x256, 2x2 waves, k64 x2, compiler-scheduled
    assert apply_opts(F16, []) == F16                     # the empty sequence is the identity
    # 2x2 waves with a 2x2 register tile is the 128x128 tile
    small = apply_opts(F16, [(L.OPT_LOCAL, 0, 16), (L.OPT_UPCAST, 0, 2), (L.OPT_UPCAST, 1, 2)])
    assert params(small)["variant"] == "1"
    # staging: TILE(reduce, 8) = k32 x 4 stages, with the asm DMAs (variant 12, 4x2 waves)
    assert params(apply_opts(F16, [(L.OPT_TILE, 2, 8), (L.OPT_VECTORIZE, 2, 4)]))["variant"] == "12"
    # the rest of the key is unchanged
    p = params(small)
    for k in ("dtype", "epi", "ta", "tb", "M", "N", "K"):
        assert p[k] == params(F16)[k]


def test_schedule_and_group_opts():
    sched = apply_opts(F16, [(L.OPT_VECTORIZE, 2, 4), (L.OPT_SCHEDULE, 0, 7)])
    assert params(sched)["variant"] == "30"              # 256x256 4x2 waves, fetch mode 7, XB
    kg = apply_opts(F16, [(L.OPT_LOCAL, 0, 16), (L.OPT_UPCAST, 0, 2), (L.OPT_UPCAST, 1, 2), (L.OPT_GROUP, 2, 2)])
    assert params(kg)["variant"] == "10"                 # 128x128, 2 k-groups, compiler-scheduled


def test_mfma_shape_opt():
    """MFMA(axis 2, 16) moves a kernel to its 16x16x32 form where one is instantiated (the asm-issued
    schedules), and MFMA(axis 2, 32) back; the compiler-scheduled class has no 16x16x32 form."""
    sched = [(L.OPT_VECTORIZE, 2, 4), (L.OPT_SCHEDULE, 0, 6)]
    assert params(apply_opts(F16, sched))["variant"] == "27"
    assert params(apply_opts(F16, sched + [(L.OPT_MFMA, 2, 16)]))["variant"] == "32"
    assert params(apply_opts(F16, sched + [(L.OPT_MFMA, 2, 16), (L.OPT_MFMA, 2, 32)]))["variant"] == "27"
    kg = [(L.OPT_LOCAL, 0, 16), (L.OPT_UPCAST, 0, 2), (L.OPT_UPCAST, 1, 2), (L.OPT_GROUP, 2, 2),
          (L.OPT_VECTORIZE, 2, 4), (L.OPT_SCHEDULE, 0, 7)]
    assert params(apply_opts(F16, kg))["variant"] == "31"
    assert params(apply_opts(F16, kg + [(L.OPT_MFMA, 2, 16)]))["variant"] == "37"
    with pytest.raises(L.AnnealHipError):
        apply_opts(F16, [(L.OPT_MFMA, 2, 16)])          # variant 3's compiler-scheduled form: no MI 16 twin
    with pytest.raises(L.AnnealHipError):
        apply_opts(F16, [(L.OPT_MFMA, 0, 16)])          # the MFMA shape is a reduce-axis opt
    assert (L.OPT_MFMA, 2, 16) in action_space(apply_opts(F16, sched))


def test_invalid_sequences_fail_closed():
    for opts in ([(L.OPT_LOCAL, 3, 16)], [(L.OPT_UPCAST, 2, 2)], [(L.OPT_TILE, 0, 8)],
                 [(L.OPT_LOCAL, 0, 32), (L.OPT_UPCAST, 0, 4)]):        # 4 waves x 4 blocks: no such tile
        with pytest.raises(L.AnnealHipError):
            apply_opts(F16, opts)
    with pytest.raises(L.AnnealHipError):
        apply_opts("tmpl:reduce;op=sum;axis=0;M=4;N=4", [(L.OPT_LOCAL, 0, 8)])   # no tunable parameters


def test_action_space_changes_the_kernel():
    acts = action_space(F16)
    assert acts and len(set(acts)) == len(acts)
    base = apply_opts(F16, [])
    for a in acts:
        k = apply_opts(F16, [a])                           # every action yields an instantiated, different kernel
        assert k != base
    assert (L.OPT_LOCAL, 0, 16) in acts and (L.OPT_LOCAL, 3, 16) not in acts
    assert action_space("tmpl:reduce;op=sum;axis=0;M=4;N=4") == []


def test_f32_tile_and_kgroups():
    k = apply_opts(F32, [(L.OPT_UPCAST, 0, 2)])
    assert params(k)["tile"] == "128"
    k = apply_opts(F32, [(L.OPT_GROUP, 2, 4)])
    assert params(k)["tile"] == "64" and params(k)["kg"] == "4"
    with pytest.raises(L.AnnealHipError):
        apply_opts(F32, [(L.OPT_UPCAST, 0, 4), (L.OPT_GROUP, 2, 4)])   # a 256 tile admits no k-groups
    acts = action_space(F32)
    assert (L.OPT_UPCAST, 0, 2) in acts and (L.OPT_GROUP, 2, 2) in acts and (L.OPT_LOCAL, 0, 8) not in acts


def test_f32_direct_to_lds_opts():
    """VECTORIZE selects the f32 direct-to-LDS kernel (key dma=i, no tile / kg / splits), TILE then sets
    its k per stage and stages in flight, UPCAST its tile; k-groups do not combine with it, and a
    (tile, stage) pair it does not instantiate fails closed."""
    k = apply_opts(F32, [(L.OPT_VECTORIZE, 2, 4)])
    assert params(k)["dma"] == "2" and "tile" not in params(k) and "kg" not in params(k)   # 64 tile, k 32 x 4
    assert params(apply_opts(F32, [(L.OPT_VECTORIZE, 2, 4), (L.OPT_TILE, 2, 32)]))["dma"] == "0"   # k 64 x 3
    assert params(apply_opts(F32, [(L.OPT_VECTORIZE, 2, 4), (L.OPT_UPCAST, 0, 2)]))["dma"] == "3"  # 128, k 32 x 4
    assert params(apply_opts(F32, [(L.OPT_VECTORIZE, 2, 4), (L.OPT_UPCAST, 1, 2), (L.OPT_TILE, 2, 16)]))["dma"] == "4"
    with pytest.raises(L.AnnealHipError):
        apply_opts(F32, [(L.OPT_VECTORIZE, 2, 4), (L.OPT_TILE, 2, 16)])      # a 64 tile with k 64 x 2: none
    with pytest.raises(L.AnnealHipError):
        apply_opts(F32, [(L.OPT_GROUP, 2, 2), (L.OPT_VECTORIZE, 2, 4)])      # k-groups stay register-staged
    with pytest.raises(L.AnnealHipError):
        apply_opts(F32, [(L.OPT_VECTORIZE, 2, 4), (L.OPT_GROUP, 2, 2)])
    acts = action_space(F32)
    assert (L.OPT_VECTORIZE, 2, 4) in acts and (L.OPT_TILE, 2, 8) not in acts   # TILE only after VECTORIZE
    dk = apply_opts(F32, [(L.OPT_VECTORIZE, 2, 4)])
    assert (L.OPT_TILE, 2, 32) in action_space(dk) and (L.OPT_GROUP, 2, 2) not in action_space(dk)
