"""CPU tests of the C-ABI boundary and the host-side operator logic.

No kernel is launched here (there is no GPU in the build container): the
library must load, export every symbol include/flash_spacetime.h declares
with the binding's signature, validate arguments before touching the
device, and report errors the way the reference's operators do.
"""

import ctypes
import re
from pathlib import Path

import pytest
import torch

import oracle
import flash_spacetime_amd
from flash_spacetime_amd import _lib
from flash_spacetime_amd import reference as spec_api
from flash_spacetime_amd.build import source_hash

HEADER = Path(__file__).resolve().parents[1] / "include" / "flash_spacetime.h"

needs_lib = pytest.mark.skipif(not _lib.LIB_PATH.exists(),
                               reason="libflash_spacetime.so not built (run flash_spacetime_amd.build)")


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(fst_\w+)\s*\(", text, flags=re.M)


def test_header_declares_expected_entry_points():
    names = set(_declared_functions())
    assert {"fst_forward", "fst_backward", "fst_forward_workspace_bytes",
            "fst_backward_workspace_bytes", "fst_supported", "fst_last_error",
            "fst_frequencies", "fst_version"} <= names
    assert names == set(_lib.SIGNATURES), "binding signatures out of sync with the header"


@needs_lib
def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    version = lib.fst_version().decode()
    assert version.startswith("flash-spacetime-gfx950 ")
    # the ABI number of the header this binding was written for (fst_backward
    # takes the forward's output before `scale`), and the build of these sources
    m = re.fullmatch(r"flash-spacetime-gfx950 \d+\.\d+\.\d+ abi (\d+) build ([0-9a-f]{12})", version)
    assert m and m.group(1) == "2", version
    assert m.group(2) == source_hash(), "the library was built from other sources than these"


@needs_lib
@pytest.mark.parametrize("c", [16, 32, 48, 64])
def test_library_frequency_ladder_equals_oracle(c):
    assert torch.equal(_lib.frequencies(c), oracle.frequencies(c))


@needs_lib
def test_supported_shapes():
    lib = _lib.load()
    for dtype in (_lib.FST_BF16, _lib.FST_F32):
        for h in (1, 4, 8, 12, 16):
            assert lib.fst_supported(dtype, h, 32, 16) == 1
            assert lib.fst_supported(dtype, h, 48, 48) == 1
    assert lib.fst_supported(_lib.FST_BF16, 8, 64, 64) == 1
    assert lib.fst_supported(_lib.FST_F32, 8, 64, 64) == 1
    assert lib.fst_supported(_lib.FST_BF16, 17, 32, 16) == 0
    assert lib.fst_supported(_lib.FST_BF16, 12, 24, 16) == 0
    assert lib.fst_supported(_lib.FST_BF16, 12, 32, 12) == 0
    assert lib.fst_supported(7, 12, 32, 16) == 0


@needs_lib
def test_workspace_queries():
    lib = _lib.load()
    fwd = lib.fst_forward_workspace_bytes(_lib.FST_BF16, 3, 256, 12, 768, 0, 32, 16)
    assert fwd >= 257 * 4 and fwd % 256 == 0
    bwd = lib.fst_backward_workspace_bytes(_lib.FST_BF16, 3, 256, 12, 768, 0, 32, 16)
    # u, w~ ([rows, H, C]) and qt ([rows, H, D], bf16 only) dominate the
    # backward scratch: linear in the number of rows, nothing O(L^2).
    rows_h = 256 * 768 * 12
    assert rows_h * (2 * 16 + 32) * 2 <= bwd < rows_h * (2 * 16 + 32) * 2 + 64 * 2 ** 20
    f32 = lib.fst_backward_workspace_bytes(_lib.FST_F32, 3, 256, 12, 768, 0, 32, 16)
    assert 2 * rows_h * 16 * 4 <= f32 < 2 * rows_h * 16 * 4 + 64 * 2 ** 20
    packed = lib.fst_backward_workspace_bytes(_lib.FST_BF16, 3 | _lib.FST_PACKED, 4096, 12, 0, 973765, 32, 16)
    assert packed > 0
    assert lib.fst_backward_workspace_bytes(_lib.FST_BF16, 3, 4, 17, 64, 0, 32, 16) == 0


@needs_lib
def test_argument_errors_are_reported_before_any_launch():
    lib = _lib.load()
    common = dict(q=None, k=None, v=None)
    rc = lib.fst_forward(9, 3, 1, 4, 8, 0, 32, 16, None, None, None, None, None, None, None, 1.0,
                         None, None, None, 0, None)
    assert rc == _lib.FST_EINVAL and "dtype" in _lib.last_error()
    rc = lib.fst_forward(0, 3, 1, 20, 8, 0, 32, 16, None, None, None, None, None, None, None, 1.0,
                         None, None, None, 0, None)
    assert rc == _lib.FST_EUNSUPPORTED and "heads" in _lib.last_error()
    rc = lib.fst_forward(0, 3, 1, 4, 8, 0, 32, 12, None, None, None, None, None, None, None, 1.0,
                         None, None, None, 0, None)
    assert rc == _lib.FST_EUNSUPPORTED and "C" in _lib.last_error()
    rc = lib.fst_forward(0, 3, 1, 4, 8, 0, 32, 16, None, None, None, None, None, None, None, 1.0,
                         None, None, None, 0, None)
    assert rc == _lib.FST_EINVAL and "null" in _lib.last_error()
    rc = lib.fst_forward(0, 3 | 64, 1, 4, 8, 0, 32, 16, None, None, None, None, None, None, None, 1.0,
                         None, None, None, 0, None)
    assert rc == _lib.FST_EINVAL and "flag" in _lib.last_error()
    # token-major is a padded layout; packed tensors are token-major already
    rc = lib.fst_forward(0, 3 | _lib.FST_PACKED | _lib.FST_TOKEN_MAJOR, 1, 4, 0, 8, 32, 16, None, None, None,
                         None, None, None, None, 1.0, None, None, None, 0, None)
    assert rc == _lib.FST_EINVAL and "TOKEN_MAJOR" in _lib.last_error()
    assert lib.fst_backward_workspace_bytes(_lib.FST_BF16, 3 | _lib.FST_TOKEN_MAJOR, 256, 12, 768, 0, 32, 16) == \
        lib.fst_backward_workspace_bytes(_lib.FST_BF16, 3, 256, 12, 768, 0, 32, 16)
    # one padded event past 2 GiB (the kernels' 32-bit offsets) is refused
    rc = lib.fst_forward(0, 3, 1, 16, 1 << 20, 0, 64, 16, None, None, None, None, None, None, None, 1.0,
                         None, None, None, 0, None)
    assert rc == _lib.FST_EUNSUPPORTED and "2^31" in _lib.last_error()
    # empty problems are valid no-ops
    assert lib.fst_forward(0, 3, 0, 4, 8, 0, 32, 16, None, None, None, None, None, None, None, 1.0,
                           None, None, None, 0, None) == _lib.FST_OK
    del common


def test_operators_refuse_cpu_tensors():
    """There is no CPU path: host tensors raise instead of falling back."""
    from flash_spacetime_amd import flash_spacetime_attention, flash_spacetime_attention_varlen

    q = torch.randn(1, 2, 8, 32)
    feats = torch.randn(1, 8, 4)
    w = torch.randn(32, 16)
    with pytest.raises(RuntimeError, match="GPU"):
        flash_spacetime_attention(q, q, q, feats, w, None, torch.tensor([8]))
    with pytest.raises(RuntimeError, match="GPU"):
        flash_spacetime_attention_varlen(q[0].transpose(0, 1), q[0].transpose(0, 1), q[0].transpose(0, 1),
                                         feats[0], w, None, torch.tensor([0, 8]))


def test_reference_backward_flag_is_refused(monkeypatch):
    from flash_spacetime_amd.forward import _FlashSpacetimeAttention

    monkeypatch.setenv("FLASH_ST_REFERENCE_BWD", "1")

    class Ctx:
        pass

    with pytest.raises(RuntimeError, match="FLASH_ST_REFERENCE_BWD"):
        _FlashSpacetimeAttention.backward(Ctx(), torch.zeros(1))


def test_package_exports_reference_names():
    for name in ("flash_spacetime_attention", "flash_spacetime_attention_varlen",
                 "spacetime_attention_reference", "spacetime_pair_features", "sinusoidal_frequencies",
                 "attention_rel_oracle_inputs", "pair_mask_bias", "float_padding_mask", "valid_row_mask",
                 "split_heads", "merge_heads", "TIME_SCALE", "SINEMB_INPUT_SCALE", "SINEMB_CLIP",
                 "SINEMB_N_FREQ"):
        assert name in flash_spacetime_amd.__all__
        assert getattr(flash_spacetime_amd, name) is not None


def test_spec_api_agrees_with_oracle():
    """The package's spec functions (pure PyTorch) equal the pinned oracle."""
    gen = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(2, 3, 9, 16, generator=gen, dtype=torch.float64) for _ in range(3))
    feats = torch.randn(2, 9, 5, generator=gen, dtype=torch.float64)
    w = torch.randn(16, 8, generator=gen, dtype=torch.float64)
    b = torch.randn(16, generator=gen, dtype=torch.float64)
    seqlens = torch.tensor([9, 4])
    mask = spec_api.float_padding_mask(spec_api.valid_row_mask(2, 9, seqlens), torch.float32)
    got = spec_api.spacetime_attention_reference(q, k, v, feats, w, b, key_padding_mask=mask)
    want = oracle.attention(q, k, v, feats, w, b, key_padding_mask=mask)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
    assert torch.equal(spec_api.pair_mask_bias(mask), oracle.pair_mask(mask))
    x = torch.randn(2, 7, 12, generator=gen)
    assert torch.equal(spec_api.merge_heads(spec_api.split_heads(x, 3)), x)


def test_mask_to_lengths_validation():
    from flash_spacetime_amd.forward import lengths_from_mask

    valid = torch.tensor([[True, True, False], [True, False, False]])
    assert torch.equal(lengths_from_mask(~valid, 3), torch.tensor([2, 1], dtype=torch.int32))
    fmask = oracle.float_padding_mask(valid, torch.float32)
    assert torch.equal(lengths_from_mask(fmask, 3), torch.tensor([2, 1], dtype=torch.int32))
    holes = torch.tensor([[True, False, True]])
    with pytest.raises(ValueError, match="front-packed"):
        lengths_from_mask(~holes, 3)


def test_ctypes_pointer_widths():
    assert ctypes.sizeof(ctypes.c_void_p) == 8
    assert ctypes.sizeof(ctypes.c_size_t) == 8


@needs_lib
@pytest.mark.parametrize("dtype,es", [(_lib.FST_BF16, 2), (_lib.FST_F32, 4)])
@pytest.mark.parametrize("h,d,c,flags", [(12, 32, 16, 3), (16, 64, 16, 3 | _lib.FST_PACKED),
                                          (16, 16, 64, 3 | _lib.FST_PACKED),
                                          (8, 64, 64, 3 | _lib.FST_PACKED | _lib.FST_QKV_INTERLEAVED),
                                          (1, 16, 16, 3)])
def test_max_event_len_is_the_32bit_offset_bound(dtype, es, h, d, c, flags):
    """The longest event the kernels take: its rows of all heads -- q, k, v
    (3 D wide interleaved) and the C-wide scratch -- span less than 2^31
    bytes, and one more token would not."""
    lib = _lib.load()
    n = lib.fst_max_event_len(dtype, flags, h, d, c)
    width = max(d * (3 if flags & _lib.FST_QKV_INTERLEAVED else 1), c)
    row = h * es * width
    assert n * row < 2 ** 31 <= (n + 1) * row
    if not flags & _lib.FST_PACKED:
        # a padded call one token past it is refused before any launch
        rc = lib.fst_forward(dtype, flags, 1, h, n + 1, 0, d, c, *([None] * 7), 1.0, None, None, None, 0, None)
        assert rc == _lib.FST_EUNSUPPORTED and "2^31" in _lib.last_error()
    assert lib.fst_max_event_len(dtype, 0, 17, d, c) == 0  # unsupported shapes report 0


def _sanitised(cu, total):
    """The work list's offsets: running maximum of cu, clamped to [0, T]."""
    out, run = [], 0
    for x in cu:
        run = max(run, x)
        out.append(min(run, total))
    return out


@pytest.mark.parametrize("seed", range(40))
def test_sanitised_offsets_fit_the_tile_slots(seed):
    """Malformed cu_seqlens (decreasing, out of range, overlapping events such
    as [0, 800, 0, 1600]) must not make the per-tile slots outnumber the
    ceil(T / 16) + B the backward workspace holds: on the sanitised offsets
    events never overlap, so their 16-row tiles are at most T / 16 + B."""
    gen = torch.Generator().manual_seed(seed)
    b = int(torch.randint(1, 40, (1,), generator=gen))
    total = int(torch.randint(0, 3000, (1,), generator=gen))
    cu = torch.randint(-200, total + 400, (b + 1,), generator=gen).tolist()
    if seed == 0:
        cu, total = [0, 800, 0, 1600], 1600
    s = _sanitised(cu, total)
    assert all(0 <= a <= e <= total for a, e in zip(s, s[1:]))
    tiles = sum(-(-(e - a) // 16) for a, e in zip(s, s[1:]))
    assert tiles <= -(-total // 16) + b
    naive = sum(-(-max(0, min(e, total) - max(0, min(a, total))) // 16) for a, e in zip(cu, cu[1:]))
    if seed == 0:
        assert naive > -(-total // 16) + b  # the advisor's overlap case overran before sanitising


@needs_lib
def test_every_head_and_channel_width_supported():
    """Both dtypes take every (D, C) in {16, 32, 48, 64}^2 at every head count
    one call covers (float32 at D = C = 64: up to 8), including float32 with
    D = 16 and C >= 48."""
    lib = _lib.load()
    for dt in (_lib.FST_F32, _lib.FST_BF16):
        for d in (16, 32, 48, 64):
            for c in (16, 32, 48, 64):
                for h in (1, 4, 8):
                    assert lib.fst_supported(dt, h, d, c) == 1, (dt, h, d, c)
