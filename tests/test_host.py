"""Host-side checks that need no GPU: the C ABI library loads and exports what the header
declares, its argument validation rejects bad calls before launching anything, the Python
boundary raises the reference's errors, and the workload bookkeeping is right."""

import ctypes
import math
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

from flicker_amd import _lib, kernels, loader, rope, workloads
from oracle import path as P

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "flicker_hip.h")).read()
    return sorted(set(re.findall(r"\b(flk_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built: run python -m flicker_amd.build")
    return _lib.lib()


def test_library_exports_every_declared_symbol(lib):
    syms = declared_symbols()
    assert syms, "no declarations found in include/flicker_hip.h"
    assert sorted(_lib.SIGNATURES) == syms
    for name in syms:
        assert hasattr(lib, name), name
    assert lib.flk_abi_version() == _lib.ABI_VERSION


def test_header_is_plain_c():
    """include/flicker_hip.h is the FFI boundary (ctypes here; cgo or a C caller elsewhere): it
    must parse as C99, not only as C++."""
    import shutil
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler on this host")
    proc = subprocess.run([cc, "-fsyntax-only", "-Wall", "-Wextra", "-Werror", "-std=c99", "-x", "c",
                           os.path.join(ROOT, "include", "flicker_hip.h")], capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr


def test_status_strings(lib):
    for code in (_lib.FLK_OK, _lib.FLK_E_INVALID, _lib.FLK_E_ALIGN, _lib.FLK_E_UNSUPPORTED, _lib.FLK_E_SCRATCH):
        assert _lib.status_string(code)
    assert "unsupported" in _lib.status_string(_lib.FLK_E_UNSUPPORTED)


FAKE = 0x10000  # a 16-byte aligned, never dereferenced address: every call below fails validation first


def test_attend_validation(lib):
    f = lib.flk_attend
    assert f(FAKE, FAKE, FAKE, FAKE, 1, 24, 4608, 64, None) == _lib.FLK_E_UNSUPPORTED
    assert f(FAKE, FAKE, FAKE, FAKE, -1, 24, 4608, 128, None) == _lib.FLK_E_INVALID
    assert f(FAKE + 8, FAKE, FAKE, FAKE, 1, 24, 4608, 128, None) == _lib.FLK_E_ALIGN
    assert f(None, FAKE, FAKE, FAKE, 1, 24, 4608, 128, None) == _lib.FLK_E_INVALID
    assert f(FAKE, FAKE, FAKE, FAKE, 0, 24, 4608, 128, None) == _lib.FLK_OK       # empty: nothing launched
    # positions up to a tile past the end must stay within int
    assert f(FAKE, FAKE, FAKE, FAKE, 1, 1, 2 ** 31 - 1, 128, None) == _lib.FLK_E_INVALID
    assert f(FAKE, FAKE, FAKE, FAKE, 1, 1, 2 ** 31 - 256, 128, None) == _lib.FLK_E_INVALID
    g = lib.flk_attend_to
    hd = 24 * 128
    assert g(FAKE, FAKE, FAKE, FAKE, 1, 24, 4608, 128, 4608 * hd, 128, hd + 2, None) == _lib.FLK_E_ALIGN
    assert g(FAKE, FAKE, FAKE, FAKE + 4, 1, 24, 4608, 128, 4608 * hd, 128, hd, None) == _lib.FLK_E_ALIGN
    assert g(FAKE, FAKE, FAKE, FAKE, 1, 24, 4608, 128, 4608 * hd, 128, 64, None) == _lib.FLK_E_INVALID
    assert g(FAKE, FAKE, FAKE, FAKE, 1, 24, 4608, 64, 4608 * hd, 128, hd, None) == _lib.FLK_E_UNSUPPORTED


def test_attend_split_plan_and_validation(lib):
    """flk_attend_plan splits only grids below 192 blocks of 256 queries, into as many key
    ranges as fill 256 CUs once with at least 512 keys each; flk_attend_split_to rejects bad
    split counts and short or misaligned workspaces before launching anything."""
    cases = {(1, 24, 4608): 1, (1, 12, 4608): 1, (1, 24, 1536): 1, (1, 6, 4608): 2, (1, 3, 4608): 4,
             (1, 1, 4608): 9, (1, 2, 257): 1, (1, 1, 64): 1, (0, 3, 4608): 1}
    for (b, h, length), want in cases.items():
        splits, nbytes = _lib.attend_plan(b, h, length)
        assert splits == want, (b, h, length, splits)
        assert nbytes == (splits * b * h * -(-length // 256) * 512 * 65 * 4 if splits > 1 else 0)
    f = lib.flk_attend_split_to
    hd, need = 3 * 128, 4 * 3 * 18 * 512 * 65 * 4
    args = (FAKE, FAKE, FAKE, FAKE, 1, 3, 4608, 128, 4608 * hd, 128, hd)
    assert f(*args, 0, FAKE, need, None) == _lib.FLK_E_INVALID           # no ranges
    assert f(*args, 19, FAKE, 10 ** 9, None) == _lib.FLK_E_INVALID       # more ranges than key groups
    assert f(*args, 4, FAKE, need - 1, None) == _lib.FLK_E_INVALID       # short workspace
    assert f(*args, 4, None, need, None) == _lib.FLK_E_INVALID
    assert f(*args, 4, FAKE + 4, need, None) == _lib.FLK_E_ALIGN
    assert f(FAKE, FAKE, FAKE, FAKE, 1, 0, 4608, 128, 0, 128, hd, 4, None, 0, None) == _lib.FLK_OK   # empty
    with pytest.raises(_lib.HipKernelError):
        _lib.check(lib.flk_attend_plan(1, -1, 10, ctypes.byref(ctypes.c_int()), ctypes.byref(ctypes.c_int64())),
                   "flk_attend_plan")


def test_attend_balanced_plan_and_validation(lib):
    """flk_attend_balanced_plan prefers the balanced launch only where every XCD has a full
    round of 32 tiles, at most 16 are left over on the fullest XCD, and each CU's share of
    their keys is at least 16 key tiles (Klein 1024^2: 54 tiles per XCD, 22 left over -> the
    rounds launch; 2048^2: 198 -> 6 left over -> balanced; 1536x640: 19 left over -> rounds;
    48 heads at 1536 tokens: 4 left over, shares of 3 key tiles -> rounds; 512^2: 18 tiles,
    no full round); its workspace does not depend on the shape.  flk_attend_balanced_to
    rejects short or misaligned workspaces before launching anything."""
    ws = 2 * 256 * (8 * 1024 * 16 + 8 * 64 * 4)
    cases = {(1, 24, 4608): 0, (4, 24, 4608): 0, (1, 24, 16896): 256, (1, 24, 4352): 0, (1, 32, 4608): 256,
             (2, 24, 4608): 256, (3, 7, 4100): 256, (1, 48, 1536): 0,
             (1, 24, 6400): 256, (1, 128, 512): 0, (1, 6, 4608): 0, (1, 24, 1536): 0, (1, 40, 1000): 0,
             (0, 3, 4608): 0}
    for (b, h, length), want in cases.items():
        grid, nbytes, counters = _lib.attend_balanced_plan(b, h, length)
        assert grid == want, (b, h, length, grid)
        assert (nbytes, counters) == (ws + 4 * 256, ws)
    f = lib.flk_attend_balanced_to
    hd = 24 * 128
    args = (FAKE, FAKE, FAKE, FAKE, 1, 24, 4608, 128, 4608 * hd, 128, hd)
    assert f(*args, FAKE, ws + 4 * 256 - 1, None) == _lib.FLK_E_INVALID
    assert f(*args, None, ws + 4 * 256, None) == _lib.FLK_E_INVALID
    assert f(*args, FAKE + 8, ws + 4 * 256, None) == _lib.FLK_E_ALIGN
    assert f(FAKE, FAKE, FAKE, FAKE, 1, 24, 4608, 64, 4608 * hd, 128, hd, FAKE, ws + 4 * 256, None) == \
        _lib.FLK_E_UNSUPPORTED
    assert f(FAKE, FAKE, FAKE, FAKE, 0, 24, 4608, 128, 4608 * hd, 128, hd, None, 0, None) == _lib.FLK_OK  # empty
    with pytest.raises(_lib.HipKernelError):
        _lib.check(lib.flk_attend_balanced_plan(1, -1, 10, ctypes.byref(ctypes.c_int()), ctypes.byref(ctypes.c_int64()),
                                                ctypes.byref(ctypes.c_int64())), "flk_attend_balanced_plan")


def test_attend_kernel_names(lib):
    """flk_attend_kernel names what flk_attend launches: 192-query tiles where both tilings fit
    the 256 CUs in one round, whole rounds plus 192-query leftovers where every XCD has a full
    round and its leftover tiles fit one round of 192-query tiles, else one block per tile."""
    cases = {(1, 24, 1536): "attend_tile192_kernel", (1, 3, 4608): "attend_tile192_kernel",
             (1, 1, 1): "attend_tile192_kernel", (1, 24, 4608): "attend_rounds_kernel",
             (1, 24, 4352): "attend_rounds_kernel", (1, 48, 1536): "attend_rounds_kernel",
             (1, 128, 512): "attend_kernel", (1, 64, 1024): "attend_kernel", (0, 24, 4608): "",
             (1, 24, 0): ""}
    for shape, want in cases.items():
        assert _lib.attend_kernel_name(*shape) == want, (shape, _lib.attend_kernel_name(*shape))


def test_attend_split_static_validation(lib):
    """flk_attend_split_static_to refuses, before launching anything, split counts out of range
    and calls whose partials would not fit its fixed buffer; every split flk_attend_plan picks
    does fit."""
    f = lib.flk_attend_split_static_to
    hd = 3 * 128
    args = (FAKE, FAKE, FAKE, FAKE, 1, 3, 4608, 128, 4608 * hd, 128, hd)
    assert f(*args, 0, None) == _lib.FLK_E_INVALID
    assert f(*args, 19, None) == _lib.FLK_E_INVALID
    assert f(FAKE, FAKE, FAKE, FAKE, 1, 24, 16896, 128, 0, 16896 * 128, 128, 2, None) == _lib.FLK_E_SCRATCH
    assert f(FAKE, FAKE, FAKE, FAKE, 1, 2, 4608, 128, 0, 4608 * 128, 128, 8, None) == _lib.FLK_E_SCRATCH
    assert f(FAKE, FAKE, FAKE, FAKE + 4, 1, 3, 4608, 128, 0, 4608 * 128, 128, 4, None) == _lib.FLK_E_ALIGN
    assert "scratch" in _lib.status_string(_lib.FLK_E_SCRATCH)
    header = open(os.path.join(ROOT, "include", "flicker_hip.h")).read()
    assert int(re.search(r"#define FLK_ATTEND_STATIC_SCRATCH_BYTES (\d+)", header).group(1)) == \
        _lib.ATTEND_STATIC_SCRATCH_BYTES == 256 * 512 * 65 * 4
    for b in (1, 2):
        for h in range(1, 25):
            for length in (64, 257, 1536, 4352, 4608, 16896):
                _, nbytes = _lib.attend_plan(b, h, length)
                assert nbytes <= _lib.ATTEND_STATIC_SCRATCH_BYTES, (b, h, length, nbytes)


def test_qk_prep_validation(lib):
    f = lib.flk_qk_prep
    args = dict(qkv=FAKE, bs=4608 * 9216, rs=9216, cos=FAKE, sin=FAKE, ts=128, qs=FAKE, ks=FAKE, f32=0,
                gain=1.0, b=1, l=4608, h=24, d=128, q=FAKE, k=FAKE, v=FAKE, ol=4608, oo=0, st=None)

    def call(**kw):
        a = dict(args, **kw)
        return f(*a.values())

    assert call(d=64) == _lib.FLK_E_UNSUPPORTED
    assert call(oo=1) == _lib.FLK_E_INVALID                 # out_offset + L > out_length
    assert call(l=2 ** 31 - 1, ol=2 ** 31 - 1) == _lib.FLK_E_INVALID   # last block's token index past int
    assert call(rs=9000) == _lib.FLK_E_INVALID              # row shorter than 3*H*D
    assert call(rs=9220) == _lib.FLK_E_ALIGN                # row stride not a multiple of 8
    assert call(q=FAKE + 4) == _lib.FLK_E_ALIGN
    assert call(l=0) == _lib.FLK_OK


def test_qk_prep_f32_validation(lib):
    """flk_qk_prep_f32 (the plain branch with float32 scales) shares flk_qk_prep's checks:
    head width, strides, alignment, table arguments; empty problems launch nothing."""
    f = lib.flk_qk_prep_f32
    hd = 3 * 24 * 128

    def call(**kw):
        a = dict(qkv=FAKE, bs=100 * hd, rs=hd, cos=FAKE, sin=FAKE, ts=128, qs=FAKE, ks=FAKE, b=1, n=100, h=24,
                 d=128, q=FAKE, k=FAKE, v=FAKE, ol=100, oo=0)
        a.update(kw)
        return f(a["qkv"], a["bs"], a["rs"], a["cos"], a["sin"], a["ts"], a["qs"], a["ks"], a["b"], a["n"],
                 a["h"], a["d"], a["q"], a["k"], a["v"], a["ol"], a["oo"], None)

    assert call(d=64) == _lib.FLK_E_UNSUPPORTED
    assert call(rs=hd - 8) == _lib.FLK_E_INVALID
    assert call(ts=64) == _lib.FLK_E_INVALID
    assert call(cos=None) == _lib.FLK_E_INVALID
    assert call(q=FAKE + 4) == _lib.FLK_E_ALIGN
    assert call(ts=130) == _lib.FLK_E_ALIGN
    assert call(oo=1) == _lib.FLK_E_INVALID
    assert call(n=0) == _lib.FLK_OK and call(b=0) == _lib.FLK_OK


def test_qk_prep_ids_validation(lib):
    f = lib.flk_qk_prep_ids
    args = dict(qkv=FAKE, bs=4608 * 9216, rs=9216, ids=FAKE, ids_rs=4, n_axes=4,
                axes=_lib.int_array([32, 32, 32, 32]), theta=2000.0, qs=FAKE, ks=FAKE, f32=0, gain=1.0,
                b=1, l=4608, h=24, d=128, q=FAKE, k=FAKE, v=FAKE, ol=4608, oo=0, st=None)

    def call(**kw):
        a = dict(args, **kw)
        return f(*a.values())

    assert call(d=64) == _lib.FLK_E_UNSUPPORTED
    assert call(axes=_lib.int_array([32, 32, 32, 30])) == _lib.FLK_E_INVALID   # sum != head_dim
    assert call(axes=_lib.int_array([32, 32, 32, 31])) == _lib.FLK_E_INVALID   # odd axis
    assert call(n_axes=9) == _lib.FLK_E_INVALID
    assert call(ids_rs=3) == _lib.FLK_E_INVALID                                # row shorter than n_axes
    assert call(ids=None) == _lib.FLK_E_INVALID
    assert call(ids=FAKE + 2) == _lib.FLK_E_ALIGN
    assert call(oo=1) == _lib.FLK_E_INVALID
    assert call(rs=9220) == _lib.FLK_E_ALIGN
    assert call(l=0) == _lib.FLK_OK
    assert call(l=0, ids=None, qkv=None) == _lib.FLK_OK                       # empty: nothing is read


def test_position_ids_python_errors():
    pos = kernels.PositionIds(torch.zeros(8, 4), 1.0)
    qkv = torch.zeros(1, 8, 3 * 24 * 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU only"):
        kernels._launch_qk_prep(qkv, torch.ones(128), torch.ones(128), pos, 24, None, 0)
    with pytest.raises(TypeError, match="Freqs or PositionIds"):
        kernels._launch_qk_prep(qkv, torch.ones(128), torch.ones(128), object(), 24, None, 0)


def test_rope_validation(lib):
    axes = _lib.int_array([32, 32, 32, 31])
    assert lib.flk_rope_lanes(FAKE, 4, 10, 4, axes, 2000.0, FAKE, FAKE, None) == _lib.FLK_E_INVALID
    axes = _lib.int_array([32] * 9)
    assert lib.flk_rope_embed(FAKE, 9, 10, 9, axes, 2000.0, FAKE, None) == _lib.FLK_E_INVALID
    assert lib.flk_lane_pair(FAKE + 4, 10, 64, FAKE, FAKE, None) == _lib.FLK_E_ALIGN


def test_row_and_score_tiles():
    assert [kernels.row_tile(n) for n in (4608, 1536, 512, 4096, 16896, 4352, 100)] == \
        [2304, 1536, 512, 512, 1536, 256, None]
    assert kernels.row_tile(4608) == P.row_tile(4608)


def test_python_errors_follow_the_reference():
    qkv = torch.zeros(1, 100, 9216, dtype=torch.bfloat16)
    f = kernels.Freqs(torch.zeros(100, 128), torch.zeros(100, 128))
    with pytest.raises(ValueError, match="qk_prep needs a row tile dividing L=100"):
        kernels.qk_prep(qkv, torch.ones(128), torch.ones(128), f, 24)
    with pytest.raises(ValueError, match="interpret"):
        kernels.qk_prep(qkv, torch.ones(128), torch.ones(128), f, 24, interpret=True)
    q = torch.zeros(1, 2, 100, 128, dtype=torch.bfloat16)
    with pytest.raises(StopIteration):
        kernels.attend(q, q, q)
    with pytest.raises(ValueError, match="does not divide"):
        kernels.attend(q, q, q, block=64)
    q = torch.zeros(1, 2, 128, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        kernels.attend(q, q, q)                              # no CPU fallback
    with pytest.raises(ValueError, match="GPU"):
        kernels.qk_prep(torch.zeros(1, 128, 9216, dtype=torch.bfloat16), torch.ones(128), torch.ones(128),
                        kernels.Freqs(torch.zeros(128, 128), torch.zeros(128, 128)), 24)


def test_qkv_prep_gate_host_side():
    """modules.py:76-80: a length with no row tile takes the plain branch, which needs pe; with
    pe it goes to the GPU kernel (so a CPU tensor is refused, there is no CPU branch)."""
    from flicker_amd import modules
    qkv = torch.zeros(1, 100, 9216, dtype=torch.bfloat16)
    f = kernels.Freqs(torch.zeros(100, 128), torch.zeros(100, 128), 1 / math.sqrt(128))
    with pytest.raises(ValueError, match="plain branch needs pe"):
        modules.qkv_prep(qkv, torch.ones(128), torch.ones(128), None, f, 24)
    pe = torch.from_numpy(P.embed_nd(np.zeros((100, 4), np.float32)))
    with pytest.raises(ValueError, match="GPU"):
        modules.qkv_prep(qkv, torch.ones(128), torch.ones(128), pe, f, 24)
    with pytest.raises(ValueError, match="broadcast"):
        modules.qkv_prep(qkv, torch.ones(128), torch.ones(128), torch.cat([pe] * 3), f, 24)
    # a double block whose stream takes the plain branch with float32 scales would hand attend
    # float32 q and k: refused up front (attend takes bf16 only), before anything is launched
    txt = torch.zeros(1, 100, 9216, dtype=torch.bfloat16)
    img = torch.zeros(1, 512, 9216, dtype=torch.bfloat16)
    joint = kernels.Freqs(torch.zeros(612, 128), torch.zeros(612, 128), 1 / math.sqrt(128))
    f32, b16 = torch.ones(128), torch.ones(128, dtype=torch.bfloat16)
    with pytest.raises(TypeError, match="text stream .* float32"):
        modules.double_attention(txt, img, (f32, f32), (b16, b16), joint, 24)


def test_logit_bound_and_check_match_oracle():
    rng = np.random.default_rng(0)
    qs, ks = rng.standard_normal((2, 5, 128)).astype(np.float32)
    np.testing.assert_allclose(kernels.logit_bound(torch.from_numpy(qs), torch.from_numpy(ks)).numpy(),
                               P.logit_bound(qs, ks), rtol=1e-6)
    for v in (1.0, 2.6, 2.7, 3.0):
        blocks = {"double_blocks": {f"{s}_attn.norm.{n}.scale": np.full((5, 128), v, np.float32)
                                    for s in ("img", "txt") for n in ("query_norm", "key_norm")},
                  "single_blocks": {f"norm.{n}.scale": np.ones((20, 128), np.float32)
                                    for n in ("query_norm", "key_norm")}}
        try:
            P.check_logit_bound(blocks)
            oracle_ok = True
        except ValueError as e:
            oracle_ok, msg = False, str(e)
        if oracle_ok:
            loader.check_logit_bound(blocks)
        else:
            with pytest.raises(ValueError) as info:
                loader.check_logit_bound(blocks)
            assert str(info.value) == msg
    assert loader.sequence_margin(15.6, 4608) > 0 and loader.sequence_margin(80.0, 16896) < 0


def test_ids_match_oracle():
    np.testing.assert_array_equal(rope.img_ids(4, 6), P.img_ids(4, 6))
    np.testing.assert_array_equal(rope.txt_ids(9), P.txt_ids(9))
    np.testing.assert_array_equal(rope.sequence_ids(5, 3, 2), P.sequence_ids(5, 3, 2))


def test_workload_bookkeeping():
    w = workloads.WORKLOADS
    assert [w[n].length for n in ("klein_512", "klein_1024", "klein_1024_b4", "klein_2048", "klein_1536x640")] == \
        [1536, 4608, 4608, 16896, 4352]
    assert w["klein_1024"].qk_prep_bytes() == 2 * 4608 * 9216 * 2 + 2 * 4608 * 128 * 4 + 2 * 128 * 2 == 174588416
    assert w["klein_1024"].attend_flops() == 4 * 24 * 4608 ** 2 * 128 == 260919263232
    assert math.isclose(workloads.q_gain(w["klein_1024"]), 1 / math.sqrt(128))


def test_stress_channels_and_scales():
    w = workloads.Workload("t", 1, 4, 2, 2, stress_fraction=0.05)
    plain = workloads.Workload("t", 1, 4, 2, 2)
    a, b = workloads.make_qkv(w).float(), workloads.make_qkv(plain).float()
    ratio = (a / torch.where(b == 0, torch.ones_like(b), b))
    scaled = ((ratio - 8).abs() < 0.1).all(dim=(0, 1))
    assert int(scaled.sum()) == round(0.05 * 9216)
    qs, ks = workloads.make_scales(w)
    assert qs.dtype == torch.bfloat16 and abs(float(qs.float().mean()) - 1) < 0.02


def test_cpu_baseline_matches_oracle_plain_path():
    from oracle import cpu_baseline as cb
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn(1, 96, 3 * 2 * 128, generator=g).to(torch.bfloat16)
    qs = (1 + 0.05 * torch.randn(128, generator=g)).to(torch.bfloat16)
    ks = (1 + 0.05 * torch.randn(128, generator=g)).to(torch.bfloat16)
    ids = P.sequence_ids(32, 8, 8)
    pe = P.embed_nd(ids)
    got = cb.plain_attention(qkv, qs, ks, torch.from_numpy(pe[0, 0]), 2).numpy()
    q, k, v = P.qk_prep_plain(qkv.float().numpy(), qs.float().numpy(), ks.float().numpy(), pe, 2)
    want = P.sdpa(q, k, v)
    assert np.abs(got - want).max() <= 2e-2 and np.abs(got - want).mean() <= 2e-4


def test_operands_must_share_one_gpu():
    """Every call names its operands; they must live on one GPU, which is made current for
    the launch (a HIP launch goes to the current device, not to the operands' one)."""
    import types
    on0 = types.SimpleNamespace(device=torch.device("cuda", 0))
    on1 = types.SimpleNamespace(device=torch.device("cuda", 1))
    assert _lib.device_of(on0, None, on0) == torch.device("cuda", 0)
    with pytest.raises(ValueError, match="share one GPU"):
        _lib.device_of(on0, on1)
    with pytest.raises(ValueError, match="GPU only"):
        _lib.device_of(torch.zeros(1))
    with pytest.raises(ValueError, match="share one GPU"):
        _lib.device_of(on0, torch.zeros(1))


def test_bench_refuses_multi_gpu():
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2 and "one GPU" in proc.stderr


def test_bench_ingest_trace(tmp_path):
    """--ingest-trace: runs of >= 100 consecutive dispatches of one kernel and grid become leg
    rows (mean duration, start-to-start period); every kernel and grid gets a dispatch row."""
    cols = ["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Workgroup_Size_X", "Workgroup_Size_Y",
            "Workgroup_Size_Z", "Start_Timestamp", "End_Timestamp"]
    rows, t = [], 0
    # 120 launches of A (10 us each, every 12 us), 5 of B, 100 of A on another grid
    for name, grid, count, dur in (("void (anonymous namespace)::a_kernel<1>(int)", 2560, 120, 10_000),
                                   ("b_kernel", 256, 5, 40_000), ("void (anonymous namespace)::a_kernel<1>(int)",
                                                                   5120, 100, 20_000)):
        for _ in range(count):
            rows.append([name, grid, 1, 1, 256, 1, 1, t, t + dur])
            t += dur + 2_000
    with open(tmp_path / "run_kernel_trace.csv", "w") as f:
        f.write(",".join(cols) + "\n")
        for r in rows:
            f.write(",".join(f'"{v}"' if isinstance(v, str) else str(v) for v in r) + "\n")
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--ingest-trace", str(tmp_path)],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stderr
    lines = proc.stdout.splitlines()
    assert "| `a_kernel<1>` | 10 | 120 | 10.0 | 12.0 |" in lines
    assert "| `a_kernel<1>` | 20 | 100 | 20.0 | 22.0 |" in lines
    assert not any(line.startswith("| `b_kernel` | 1 | 5 |") and line.count("|") == 6 for line in lines)
    assert any(line.startswith("| `b_kernel` | 1 | 5 | 40.0 | 40.0 | 40.0 | 40.0 |") for line in lines)
    share_a = [line for line in lines if line.startswith("| `a_kernel<1>` | 20 | 100 | 20.0 | 20.0 |")][0]
    assert share_a.endswith(f"| {100 * 100 * 20 / (120 * 10 + 5 * 40 + 100 * 20):.2f}% |")


def test_w8a8_validation(lib):
    assert lib.flk_w8a8_gemm(FAKE, FAKE, FAKE, FAKE, 64, 192, 64, FAKE, 64, None, None) == _lib.FLK_E_UNSUPPORTED
    assert lib.flk_w8a8_gemm(FAKE, FAKE, FAKE, FAKE, 64, 256, 66, FAKE, 66, None, None) == _lib.FLK_E_UNSUPPORTED
    assert lib.flk_w8a8_gemm(FAKE, FAKE, FAKE, FAKE, 64, 256, 64, FAKE, 32, None, None) == _lib.FLK_E_INVALID
    assert lib.flk_w8a8_gemm(FAKE, FAKE, FAKE, FAKE, 64, 256, 64, FAKE + 4, 64, None, None) == _lib.FLK_E_ALIGN
    assert lib.flk_w8a8_gemm(FAKE, FAKE, FAKE, FAKE, 64, 2 ** 20, 64, FAKE, 64, None, None) == _lib.FLK_E_UNSUPPORTED
    big = 2 ** 31 - 1   # token / channel counts whose last tile would pass the int range
    assert lib.flk_w8a8_gemm(FAKE, FAKE, FAKE, FAKE, big, 256, 64, FAKE, 64, None, None) == _lib.FLK_E_INVALID
    assert lib.flk_w8a8_gemm(FAKE, FAKE, FAKE, FAKE, 64, 256, big - 3, FAKE, big - 3, None, None) == _lib.FLK_E_INVALID
    assert lib.flk_w8a8_gemm(FAKE, FAKE, FAKE, FAKE, 0, 256, 64, FAKE, 64, None, None) == _lib.FLK_OK
    assert lib.flk_quantize_act(FAKE, 3000, FAKE, 8, 3072, FAKE, FAKE, None) == _lib.FLK_E_INVALID
    assert lib.flk_quantize_act(FAKE, 3076, FAKE, 8, 3076, FAKE, FAKE, None) == _lib.FLK_E_UNSUPPORTED
    assert lib.flk_quantize_act(FAKE, 16384, FAKE, 8, 16384, FAKE, FAKE, None) == _lib.FLK_E_UNSUPPORTED
    assert lib.flk_quantize_weight(FAKE, 9216, FAKE, 3000, 9216, FAKE, FAKE, None) == _lib.FLK_E_UNSUPPORTED
    # row / column counts whose last block's index would pass the int range
    assert lib.flk_quantize_act(FAKE, 3072, FAKE, 2 ** 31 - 2, 3072, FAKE, FAKE, None) == _lib.FLK_E_INVALID
    assert lib.flk_quantize_weight(FAKE, 2 ** 31 - 8, FAKE, 3072, 2 ** 31 - 8, FAKE, FAKE, None) == \
        _lib.FLK_E_INVALID
    assert lib.flk_absmax_rows(FAKE, 4, 12, 12, FAKE, None) == _lib.FLK_E_ALIGN
    assert lib.flk_absmax_cols(FAKE, 4, 16, 8, 0, FAKE, None) == _lib.FLK_E_INVALID
    assert lib.flk_smooth_factors(FAKE, FAKE, -1, FAKE, FAKE, None) == _lib.FLK_E_INVALID
    pair = lib.flk_w8a8_qk_prep_pair

    def stream(length, offset, ptr=FAKE):
        return (ptr, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, length, offset)

    tail = (3072, 128, 0, 1.0, 1, 24, 128, FAKE, FAKE, FAKE, 4608, None)
    assert pair(*stream(512, 0), *stream(4096, 512), *tail[:6], 64, *tail[7:]) == _lib.FLK_E_UNSUPPORTED
    assert pair(*stream(-1, 0), *stream(4096, 512), *tail) == _lib.FLK_E_INVALID
    assert pair(*stream(512, 0), *stream(4096, 600), *tail) == _lib.FLK_E_INVALID     # past out_length
    assert pair(*stream(512, 0, FAKE + 4), *stream(4096, 512), *tail) == _lib.FLK_E_ALIGN
    assert pair(*stream(0, 0), *stream(0, 0), *tail) == _lib.FLK_OK                  # both empty
    qm = lib.flk_quantize_act_modulated
    assert qm(FAKE, 3072, FAKE, FAKE, 3072, 0, FAKE, 0, 3072, FAKE, FAKE, None, 0, None) == _lib.FLK_OK   # 0 tokens
    assert qm(FAKE, 3072, FAKE, FAKE, 3072, 0, FAKE, 8, 3072, FAKE, FAKE, None, 0, None) == _lib.FLK_E_INVALID


def test_w8a8_python_errors():
    from flicker_amd import w8a8
    with pytest.raises(ValueError, match="GPU"):
        w8a8.quantize_act(torch.zeros((4, 64), dtype=torch.bfloat16), torch.ones(64))
    with pytest.raises(ValueError, match="GPU"):
        w8a8.gemm(torch.zeros((4, 128), dtype=torch.int8), torch.ones(4), torch.zeros((8, 128), dtype=torch.int8),
                  torch.ones(8))


def test_projection_workload():
    p = workloads.PROJECTIONS["qkv_1024"]
    assert (p.tokens, p.hidden, p.out_features) == (4608, 3072, 9216)
    assert p.gemm_ops() == 2 * 4608 * 3072 * 9216 == 260919263232
    assert p.gemm_bytes() == 4608 * 3072 + 3072 * 9216 + 2 * 4608 * 9216
    x, w = workloads.make_projection(workloads.PROJECTIONS["qkv_512"])
    amax = x.float().abs().amax(0)
    assert int((amax > 20).sum()) == round(0.01 * 3072)          # the outlier channels
    assert abs(float(w.float().std()) - 0.02) < 1e-3
