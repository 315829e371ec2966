"""CPU tests of the kernel plans (FST_PLAN_* bits) and the tuner's host logic.

No kernel runs here: the library reports which variants are compiled for a
shape and refuses plan bits before touching the device; the tuner keys
calls by shape, names plans, and saves and loads its choices.
"""

import pytest

from flash_spacetime_amd import _lib, tune

needs_lib = pytest.mark.skipif(not _lib.LIB_PATH.exists(),
                               reason="libflash_spacetime.so not built (run flash_spacetime_amd.build)")

BF16_ALL = 0x7FF00  # every bf16 group's bits (forward, rows, cols)
F32_FWD = _lib.FST_PLAN_FWD_KC16 | _lib.FST_PLAN_FWD_KC32 | _lib.FST_PLAN_FWD_T16 | _lib.FST_PLAN_FWD_T32 \
    | _lib.FST_PLAN_FWD_T64 | _lib.FST_PLAN_FWD_W8
F32_BWD = _lib.FST_PLAN_BWD_T16 | _lib.FST_PLAN_BWD_T32 | _lib.FST_PLAN_BWD_T64 | _lib.FST_PLAN_BWD_KC16 \
    | _lib.FST_PLAN_BWD_KC32 | _lib.FST_PLAN_BWD_PASS1 | _lib.FST_PLAN_BWD_PASS2 | _lib.FST_PLAN_BWD_W8
GROUPS = [
    _lib.FST_PLAN_FWD_OCC2 | _lib.FST_PLAN_FWD_OCC3,
    _lib.FST_PLAN_ROWS_W4 | _lib.FST_PLAN_ROWS_W8 | _lib.FST_PLAN_ROWS_W8X2,
    _lib.FST_PLAN_COLS_OCC2 | _lib.FST_PLAN_COLS_OCC3,
    _lib.FST_PLAN_ROWS_KV_REG | _lib.FST_PLAN_ROWS_KV_LDS,
    _lib.FST_PLAN_FWD_KC16 | _lib.FST_PLAN_FWD_KC32,
    _lib.FST_PLAN_FWD_T16 | _lib.FST_PLAN_FWD_T32 | _lib.FST_PLAN_FWD_T64 | _lib.FST_PLAN_FWD_W8,
    _lib.FST_PLAN_BWD_T16 | _lib.FST_PLAN_BWD_T32 | _lib.FST_PLAN_BWD_T64 | _lib.FST_PLAN_BWD_W8,
    _lib.FST_PLAN_BWD_KC16 | _lib.FST_PLAN_BWD_KC32,
    _lib.FST_PLAN_BWD_PASS1 | _lib.FST_PLAN_BWD_PASS2,
]


def test_plan_groups_partition_the_mask():
    seen = 0
    for g in GROUPS:
        assert g & seen == 0 and g & ~_lib.FST_PLAN_MASK == 0
        seen |= g
    assert seen == _lib.FST_PLAN_MASK


@needs_lib
def test_plans_of_shapes():
    lib = _lib.load()
    # cfg2's shape offers every bf16 variant.
    assert lib.fst_plans(_lib.FST_BF16, 12, 32, 16) == BF16_ALL
    # Larger lane state: the two-workgroup forward and cols kernels, the
    # one-workgroup eight-wave rows kernel with register K / V, 16-key chunks.
    assert lib.fst_plans(_lib.FST_BF16, 8, 64, 64) == (
        _lib.FST_PLAN_FWD_OCC2 | _lib.FST_PLAN_FWD_KC16 | _lib.FST_PLAN_ROWS_W8 | _lib.FST_PLAN_ROWS_KV_REG
        | _lib.FST_PLAN_COLS_OCC2)
    # float32 (first-generation kernels): tile heights (eight waves per
    # 16-row tile where 8 divides the padded heads) and key chunks.
    assert lib.fst_plans(_lib.FST_F32, 8, 16, 16) == F32_FWD | F32_BWD & ~_lib.FST_PLAN_BWD_T64
    assert lib.fst_plans(_lib.FST_F32, 4, 16, 16) == F32_FWD & ~_lib.FST_PLAN_FWD_W8 | F32_BWD & ~_lib.FST_PLAN_BWD_W8
    assert lib.fst_plans(_lib.FST_F32, 8, 64, 64) == (
        _lib.FST_PLAN_FWD_KC16 | _lib.FST_PLAN_FWD_KC32 | _lib.FST_PLAN_FWD_T16 | _lib.FST_PLAN_FWD_T32
        | _lib.FST_PLAN_FWD_W8 | _lib.FST_PLAN_BWD_T16 | _lib.FST_PLAN_BWD_KC16 | _lib.FST_PLAN_BWD_PASS1
        | _lib.FST_PLAN_BWD_PASS2 | _lib.FST_PLAN_BWD_W8)
    assert lib.fst_plans(_lib.FST_BF16, 17, 32, 16) == 0
    assert lib.fst_plans(_lib.FST_BF16, 12, 24, 16) == 0
    for dtype in (_lib.FST_BF16, _lib.FST_F32):
        for h in (1, 4, 8, 12, 16):
            for d in (16, 32, 48, 64):
                for c in (16, 32, 48, 64):
                    if not lib.fst_supported(dtype, h, d, c):
                        continue
                    mask = lib.fst_plans(dtype, h, d, c)
                    if dtype == _lib.FST_BF16:
                        # every supported bf16 shape has a variant of each kernel
                        assert mask & GROUPS[0] and mask & GROUPS[1] and mask & GROUPS[2], (h, d, c, hex(mask))
                        assert mask & ~BF16_ALL == 0
                    else:
                        assert mask & GROUPS[5] and mask & GROUPS[6], (h, d, c, hex(mask))
                        assert mask & ~(F32_FWD | F32_BWD) == 0
                    # the static plan and every offered bit alone are runnable
                    assert lib.fst_plan_supported(dtype, h, d, c, 0)
                    for b in range(8, 31):
                        if mask >> b & 1:
                            assert lib.fst_plan_supported(dtype, h, d, c, 1 << b), (dtype, h, d, c, b)


@needs_lib
def test_plan_combinations():
    lib = _lib.load()
    sup = lambda *a: lib.fst_plan_supported(*a)  # noqa: E731
    bf, f32 = _lib.FST_BF16, _lib.FST_F32
    # K / V in LDS with four waves or with eight in two workgroups, not with
    # the one-workgroup eight-wave kernel
    assert sup(bf, 12, 32, 16, _lib.FST_PLAN_ROWS_W4 | _lib.FST_PLAN_ROWS_KV_LDS)
    assert sup(bf, 12, 32, 16, _lib.FST_PLAN_ROWS_W8X2 | _lib.FST_PLAN_ROWS_KV_LDS)
    assert not sup(bf, 12, 32, 16, _lib.FST_PLAN_ROWS_W8 | _lib.FST_PLAN_ROWS_KV_LDS)
    # 32-key forward chunks run at two workgroups per CU only
    assert sup(bf, 12, 32, 16, _lib.FST_PLAN_FWD_OCC2 | _lib.FST_PLAN_FWD_KC32)
    assert not sup(bf, 12, 32, 16, _lib.FST_PLAN_FWD_OCC3 | _lib.FST_PLAN_FWD_KC32)
    # K / V in LDS needs D a multiple of 32
    assert not sup(bf, 12, 16, 16, _lib.FST_PLAN_ROWS_KV_LDS)
    # float32 at D = C = 64: 32-row tiles fit with 16-key chunks only
    assert sup(f32, 8, 64, 64, _lib.FST_PLAN_FWD_T32 | _lib.FST_PLAN_FWD_KC16)
    assert not sup(f32, 8, 64, 64, _lib.FST_PLAN_FWD_T32 | _lib.FST_PLAN_FWD_KC32)
    assert not sup(f32, 8, 64, 64, _lib.FST_PLAN_FWD_T64)
    # bits of another dtype's kernels, two bits of one group, bits past the mask
    assert not sup(f32, 12, 32, 16, _lib.FST_PLAN_FWD_OCC2)
    assert not sup(bf, 12, 32, 16, _lib.FST_PLAN_FWD_T32)
    assert not sup(bf, 12, 32, 16, _lib.FST_PLAN_ROWS_W4 | _lib.FST_PLAN_ROWS_W8X2)
    assert not sup(bf, 12, 32, 16, _lib.FST_PLAN_FWD_W8)
    # eight-wave float32 tiles need the padded heads divisible by 8
    assert sup(f32, 8, 64, 64, _lib.FST_PLAN_FWD_W8) and sup(f32, 8, 64, 64, _lib.FST_PLAN_BWD_W8)
    assert not sup(f32, 12, 32, 16, _lib.FST_PLAN_FWD_W8)
    # one or two passes of the float32 rows kernel, with any fitting split
    assert sup(f32, 8, 64, 64, _lib.FST_PLAN_BWD_PASS1) and sup(f32, 8, 64, 64, _lib.FST_PLAN_BWD_PASS2)
    assert not sup(bf, 12, 32, 16, _lib.FST_PLAN_BWD_PASS1)


@needs_lib
def test_plan_bits_are_validated():
    lib = _lib.load()
    ws = lib.fst_backward_workspace_bytes
    base = ws(_lib.FST_BF16, 3, 4, 12, 64, 0, 32, 16)
    assert base > 0
    # the workspace does not depend on the plan
    for b in range(8, 31):
        if BF16_ALL >> b & 1:
            assert ws(_lib.FST_BF16, 3 | (1 << b), 4, 12, 64, 0, 32, 16) == base
    base32 = ws(_lib.FST_F32, 3, 4, 4, 64, 0, 16, 16)
    for b in range(8, 31):
        if lib.fst_plans(_lib.FST_F32, 4, 16, 16) >> b & 1:
            assert ws(_lib.FST_F32, 3 | (1 << b), 4, 4, 64, 0, 16, 16) == base32
    # two variants of one kernel knob
    rc = lib.fst_forward(0, 3 | _lib.FST_PLAN_FWD_OCC2 | _lib.FST_PLAN_FWD_OCC3, 1, 12, 8, 0, 32, 16, None,
                         None, None, None, None, None, None, 1.0, None, None, None, 0, None)
    assert rc == _lib.FST_EINVAL and "two variants" in _lib.last_error()
    rc = lib.fst_forward(1, 3 | _lib.FST_PLAN_FWD_T16 | _lib.FST_PLAN_FWD_T64, 1, 12, 8, 0, 32, 16, None,
                         None, None, None, None, None, None, 1.0, None, None, None, 0, None)
    assert rc == _lib.FST_EINVAL and "two variants" in _lib.last_error()
    # a variant not compiled for the shape (float32 has no occupancy
    # variants; D = C = 64 has no three-workgroup bf16 forward)
    rc = lib.fst_forward(1, 3 | _lib.FST_PLAN_FWD_OCC2, 1, 12, 8, 0, 32, 16, None, None, None, None, None,
                         None, None, 1.0, None, None, None, 0, None)
    assert rc == _lib.FST_EUNSUPPORTED and "plan" in _lib.last_error()
    rc = lib.fst_forward(0, 3 | _lib.FST_PLAN_FWD_OCC3, 1, 8, 8, 0, 64, 64, None, None, None, None, None,
                         None, None, 1.0, None, None, None, 0, None)
    assert rc == _lib.FST_EUNSUPPORTED and "plan" in _lib.last_error()
    assert ws(_lib.FST_BF16, 3 | _lib.FST_PLAN_ROWS_W4, 4, 8, 64, 0, 64, 64) == 0
    # bits past the plan field are unknown flags
    rc = lib.fst_forward(0, 3 | -(1 << 31), 1, 12, 8, 0, 32, 16, None, None, None, None, None, None, None,
                         1.0, None, None, None, 0, None)
    assert rc == _lib.FST_EINVAL and "flag" in _lib.last_error()


def test_shape_key_buckets():
    b = ("gfx950", "v1")
    padded = (0, 3, 256, 12, 768, 0, 32, 16)
    assert tune.shape_key("fwd", padded, b) == ("gfx950", "v1", "fwd", 0, 12, 32, 16, 3, 9, 10)
    # plan bits do not enter the key; batches of similar size share it
    assert tune.shape_key("fwd", (0, 3 | (1 << 9), 300, 12, 700, 0, 32, 16), b) == tune.shape_key("fwd", padded, b)
    assert tune.shape_key("fwd", (0, 3, 256, 12, 1100, 0, 32, 16), b) != tune.shape_key("fwd", padded, b)
    packed = (0, 3 | _lib.FST_PACKED, 4096, 12, 0, 973765, 32, 16)
    assert tune.shape_key("bwd", packed, b) == ("gfx950", "v1", "bwd", 0, 12, 32, 16, 3 | _lib.FST_PACKED, 20, 13)
    # another architecture or library build keys apart
    assert tune.shape_key("fwd", padded, ("gfx942", "v1")) != tune.shape_key("fwd", padded, b)
    assert tune.shape_key("fwd", padded, ("gfx950", "v2")) != tune.shape_key("fwd", padded, b)


def test_plan_names_and_fixed_plan():
    assert tune.plan_names(0) is None
    assert tune.plan_names(_lib.FST_PLAN_FWD_OCC3 | _lib.FST_PLAN_ROWS_W8 | _lib.FST_PLAN_COLS_OCC2) == \
        "fwd:occ3 rows:w8 cols:occ2"
    dims = (0, 3, 4, 12, 64, 0, 32, 16)
    never = lambda *a: pytest.fail("a fixed plan must not time anything")  # noqa: E731
    with tune.fixed_plan(_lib.FST_PLAN_FWD_OCC2 | _lib.FST_PLAN_ROWS_W8):
        assert tune.forward_plan(dims, never) == _lib.FST_PLAN_FWD_OCC2
        assert tune.backward_plan(dims, never) == _lib.FST_PLAN_ROWS_W8
    with pytest.raises(ValueError):
        with tune.fixed_plan(1):
            pass


def test_plan_names_cover_every_bit():
    for b in range(8, 31):
        assert tune.plan_names(1 << b), b
    assert tune.plan_names(_lib.FST_PLAN_ROWS_W8X2 | _lib.FST_PLAN_ROWS_KV_LDS | _lib.FST_PLAN_FWD_KC32) == \
        "fwd:kc32 rows:w8x2 rows:kvlds"


@needs_lib
def test_disabled_tuner_uses_the_static_plan():
    tune.clear()
    tune.set_autotune(False)
    never = lambda *a: pytest.fail("tuning is off")  # noqa: E731
    dims = (0, 3, 4, 12, 64, 0, 32, 16)
    assert tune.forward_plan(dims, never) == 0
    assert tune.backward_plan(dims, never) == 0
    assert tune.chosen() == {}
    # a choice made while tuning was on is not used while it is off
    tune._cache[tune.shape_key("fwd", dims)] = _lib.FST_PLAN_FWD_OCC2
    assert tune.forward_plan(dims, never) == 0
    tune.clear()


@needs_lib
def test_tile_arguments_map_to_plans():
    bf, f32 = _lib.FST_BF16, _lib.FST_F32
    p = tune.plan_from_tiles
    assert p(bf, 12, 32, 16, "fwd") is None  # nothing given: the library's choice
    # bf16 forward: block_n picks the key chunk; block_m has one height (16)
    assert p(bf, 12, 32, 16, "fwd", block_n=32) == _lib.FST_PLAN_FWD_KC32
    assert p(bf, 12, 32, 16, "fwd", block_n=64) == _lib.FST_PLAN_FWD_KC32
    assert p(bf, 12, 32, 16, "fwd", block_n=16) == _lib.FST_PLAN_FWD_KC16
    assert p(bf, 12, 32, 16, "fwd", block_m=64) == 0
    # ... where 32-key chunks are not compiled, the nearest offered value
    assert p(bf, 8, 64, 64, "fwd", block_n=32) == _lib.FST_PLAN_FWD_KC16
    # bf16 backward: num_warps picks the rows kernel's waves
    assert p(bf, 12, 32, 16, "bwd", num_warps=4) == _lib.FST_PLAN_ROWS_W4
    assert p(bf, 12, 32, 16, "bwd", num_warps=8) == _lib.FST_PLAN_ROWS_W8X2
    assert p(bf, 8, 64, 64, "bwd", num_warps=8) == _lib.FST_PLAN_ROWS_W8
    # float32: block_m the tile height, block_n the chunk
    assert p(f32, 4, 16, 16, "fwd", block_m=32, block_n=32) == _lib.FST_PLAN_FWD_T32 | _lib.FST_PLAN_FWD_KC32
    assert p(f32, 4, 16, 16, "bwd", block_m=64, block_n=16) == _lib.FST_PLAN_BWD_T64 | _lib.FST_PLAN_BWD_KC16
    assert p(f32, 4, 16, 16, "fwd", block_m=64, block_n=32) == _lib.FST_PLAN_FWD_T64  # 64 x 32 does not fit
    # float32: num_warps=8 asks for the eight-wave 16-row tile, 4 for four
    assert p(f32, 8, 64, 64, "fwd", num_warps=8) == _lib.FST_PLAN_FWD_W8
    assert p(f32, 8, 64, 64, "bwd", block_m=16, num_warps=8) == _lib.FST_PLAN_BWD_W8
    assert p(f32, 8, 64, 64, "bwd", num_warps=4) == _lib.FST_PLAN_BWD_T16
    assert p(f32, 8, 64, 64, "fwd", block_m=32, num_warps=8) == _lib.FST_PLAN_FWD_T32
    assert p(f32, 12, 32, 16, "fwd", num_warps=8) == _lib.FST_PLAN_FWD_T16  # 8 does not divide 12
    # a combination not compiled drops block_n (then block_m)
    assert p(f32, 8, 64, 64, "fwd", block_m=32, block_n=32) == _lib.FST_PLAN_FWD_T32
    assert p(f32, 8, 64, 64, "fwd", block_m=64) == _lib.FST_PLAN_FWD_T32
    with pytest.raises(ValueError):
        with tune.tile_request(block_m=0):
            pass
    with pytest.raises(ValueError):
        with tune.tile_request(block_n=16.0):
            pass
    never = lambda *a: pytest.fail("tile arguments are not timed")  # noqa: E731
    with tune.fixed_plan(_lib.FST_PLAN_FWD_OCC3), tune.tile_request(block_n=32):
        assert tune.forward_plan((0, 3, 4, 12, 64, 0, 32, 16), never) == _lib.FST_PLAN_FWD_KC32


def test_save_and_load(tmp_path):
    tune.clear()
    tune._cache[tune.shape_key("fwd", (0, 3, 4, 12, 64, 0, 32, 16))] = _lib.FST_PLAN_FWD_OCC2
    path = tmp_path / "plans.json"
    tune.save(str(path))
    saved = tune.chosen()
    tune.clear()
    tune.load(str(path))
    assert tune.chosen() == saved
    tune.clear()


@needs_lib
def test_head_groups():
    from flash_spacetime_amd.forward import head_groups

    bf, f32 = _lib.FST_BF16, _lib.FST_F32
    assert head_groups(bf, 12, 32, 16) == [(0, 12)]
    assert head_groups(bf, 16, 64, 64) == [(0, 16)]
    assert head_groups(bf, 24, 32, 16) == [(0, 12), (12, 24)]
    assert head_groups(bf, 17, 32, 16) == [(0, 8), (8, 17)]
    assert head_groups(bf, 64, 16, 16) == [(0, 16), (16, 32), (32, 48), (48, 64)]
    # float32 at D = C = 64 has kernels up to 8 heads (LDS)
    assert head_groups(f32, 8, 64, 64) == [(0, 8)]
    assert head_groups(f32, 12, 64, 64) == [(0, 6), (6, 12)]
    for heads in range(1, 70):
        groups = head_groups(bf, heads, 48, 32)
        assert groups[0][0] == 0 and groups[-1][1] == heads
        sizes = [h1 - h0 for h0, h1 in groups]
        assert max(sizes) <= 16 and max(sizes) - min(sizes) <= 1
        assert all(a[1] == b[0] for a, b in zip(groups, groups[1:]))
    with pytest.raises(ValueError):
        head_groups(bf, 12, 24, 16)


def test_cache_file_round_trip(tmp_path, monkeypatch):
    """FST_AUTOTUNE_CACHE: a new choice is written to the file, and a fresh
    cache reads it back instead of timing."""
    path = str(tmp_path / "plans.json")
    dims = (0, 3, 4, 12, 64, 0, 32, 16)
    monkeypatch.setattr(tune, "_cache_path", path)
    monkeypatch.setattr(tune, "_cache_loaded", False)
    monkeypatch.setattr(tune, "_enabled", True)
    monkeypatch.setattr(tune, "_usable", lambda: True)
    monkeypatch.setattr(tune, "_fastest", lambda run, cands, base, what: _lib.FST_PLAN_FWD_OCC2)
    tune.clear()
    assert tune.forward_plan(dims, None) == _lib.FST_PLAN_FWD_OCC2
    tune.clear()
    monkeypatch.setattr(tune, "_cache_loaded", False)
    monkeypatch.setattr(tune, "_fastest", lambda *a: pytest.fail("a cached choice must not be timed"))
    assert tune.forward_plan(dims, None) == _lib.FST_PLAN_FWD_OCC2
    tune.clear()


def test_cache_file_merges_writers(tmp_path):
    """Two processes writing one FST_AUTOTUNE_CACHE keep each other's choices."""
    path = str(tmp_path / "plans.json")
    build = ("gfx950", "v1")
    key_a = tune.shape_key("fwd", (0, 3, 4, 12, 64, 0, 32, 16), build)
    key_b = tune.shape_key("bwd", (0, 3, 8, 12, 64, 0, 32, 16), build)
    tune.clear()
    tune._cache[key_a] = _lib.FST_PLAN_FWD_OCC2
    tune.save(path)  # process A
    tune.clear()
    tune._cache[key_b] = _lib.FST_PLAN_ROWS_W4  # process B, which never read A's choice
    tune.save(path)
    tune.clear()
    tune.load(path)
    assert tune.chosen() == {key_a: _lib.FST_PLAN_FWD_OCC2, key_b: _lib.FST_PLAN_ROWS_W4}
    tune.clear()
