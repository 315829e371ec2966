"""CPU tests of the kernel plans (FST_PLAN_* bits) and the tuner's host logic.

No kernel runs here: the library reports which variants are compiled for a
shape and refuses plan bits before touching the device; the tuner keys
calls by shape, names plans, and saves and loads its choices.
"""

import pytest

from flash_spacetime_amd import _lib, tune

needs_lib = pytest.mark.skipif(not _lib.LIB_PATH.exists(),
                               reason="libflash_spacetime.so not built (run flash_spacetime_amd.build)")

ALL = 0x3F00


@needs_lib
def test_plans_of_shapes():
    lib = _lib.load()
    # cfg2's shape offers both variants of every kernel.
    assert lib.fst_plans(_lib.FST_BF16, 12, 32, 16) == ALL
    # Larger lane state: the two-workgroup forward and cols kernels and the
    # eight-wave rows kernel only.
    assert lib.fst_plans(_lib.FST_BF16, 8, 64, 64) == (_lib.FST_PLAN_FWD_OCC2 | _lib.FST_PLAN_ROWS_W8
                                                        | _lib.FST_PLAN_COLS_OCC2)
    # float32 runs one static variant; unsupported shapes have none.
    assert lib.fst_plans(_lib.FST_F32, 12, 32, 16) == 0
    assert lib.fst_plans(_lib.FST_BF16, 17, 32, 16) == 0
    assert lib.fst_plans(_lib.FST_BF16, 12, 24, 16) == 0
    for h in (1, 4, 8, 12, 16):
        for d in (16, 32, 48, 64):
            for c in (16, 32, 48, 64):
                mask = lib.fst_plans(_lib.FST_BF16, h, d, c)
                # every supported bf16 shape has at least one variant of each kernel
                assert mask & 0x300 and mask & 0xC00 and mask & 0x3000, (h, d, c, hex(mask))
                assert mask & ~ALL == 0


@needs_lib
def test_plan_bits_are_validated():
    lib = _lib.load()
    ws = lib.fst_backward_workspace_bytes
    base = ws(_lib.FST_BF16, 3, 4, 12, 64, 0, 32, 16)
    assert base > 0
    for bit in (1 << 8, 1 << 9, 1 << 10, 1 << 11, 1 << 12, 1 << 13):
        assert ws(_lib.FST_BF16, 3 | bit, 4, 12, 64, 0, 32, 16) == base
    # two variants of one kernel
    rc = lib.fst_forward(0, 3 | _lib.FST_PLAN_FWD_OCC2 | _lib.FST_PLAN_FWD_OCC3, 1, 12, 8, 0, 32, 16, None,
                         None, None, None, None, None, None, 1.0, None, None, None, 0, None)
    assert rc == _lib.FST_EINVAL and "two variants" in _lib.last_error()
    # a variant not compiled for the shape (fp32 has none; D = C = 64 has no
    # three-workgroup forward)
    rc = lib.fst_forward(1, 3 | _lib.FST_PLAN_FWD_OCC2, 1, 12, 8, 0, 32, 16, None, None, None, None, None,
                         None, None, 1.0, None, None, None, 0, None)
    assert rc == _lib.FST_EUNSUPPORTED and "plan" in _lib.last_error()
    rc = lib.fst_forward(0, 3 | _lib.FST_PLAN_FWD_OCC3, 1, 8, 8, 0, 64, 64, None, None, None, None, None,
                         None, None, 1.0, None, None, None, 0, None)
    assert rc == _lib.FST_EUNSUPPORTED and "plan" in _lib.last_error()
    assert ws(_lib.FST_BF16, 3 | _lib.FST_PLAN_ROWS_W4, 4, 8, 64, 0, 64, 64) == 0
    # bits past the plan field are unknown flags
    rc = lib.fst_forward(0, 3 | (1 << 14), 1, 12, 8, 0, 32, 16, None, None, None, None, None, None, None,
                         1.0, None, None, None, 0, None)
    assert rc == _lib.FST_EINVAL and "flag" in _lib.last_error()


def test_shape_key_buckets():
    padded = (0, 3, 256, 12, 768, 0, 32, 16)
    assert tune.shape_key("fwd", padded) == ("fwd", 0, 12, 32, 16, 3, 9, 10)
    # plan bits do not enter the key; batches of similar size share it
    assert tune.shape_key("fwd", (0, 3 | (1 << 9), 300, 12, 700, 0, 32, 16)) == tune.shape_key("fwd", padded)
    assert tune.shape_key("fwd", (0, 3, 256, 12, 1100, 0, 32, 16)) != tune.shape_key("fwd", padded)
    packed = (0, 3 | _lib.FST_PACKED, 4096, 12, 0, 973765, 32, 16)
    assert tune.shape_key("bwd", packed) == ("bwd", 0, 12, 32, 16, 3 | _lib.FST_PACKED, 20, 13)


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


def test_disabled_tuner_uses_the_static_plan():
    tune.clear()
    tune.set_autotune(False)
    never = lambda *a: pytest.fail("tuning is off")  # noqa: E731
    assert tune.forward_plan((0, 3, 4, 12, 64, 0, 32, 16), never) == 0
    assert tune.backward_plan((0, 3, 4, 12, 64, 0, 32, 16), never) == 0
    assert tune.chosen() == {}


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
    monkeypatch.setattr(tune, "_usable", lambda: True)
    monkeypatch.setattr(tune, "_fastest", lambda run, cands, base, what: _lib.FST_PLAN_FWD_OCC2)
    monkeypatch.setattr(tune, "plans", lambda *a: 0x3F00)
    tune.clear()
    assert tune.forward_plan(dims, None) == _lib.FST_PLAN_FWD_OCC2
    tune.clear()
    monkeypatch.setattr(tune, "_cache_loaded", False)
    monkeypatch.setattr(tune, "_fastest", lambda *a: pytest.fail("a cached choice must not be timed"))
    assert tune.forward_plan(dims, None) == _lib.FST_PLAN_FWD_OCC2
    tune.clear()
