"""int8 SmoothQuant W8A8 QKV projection on the GPU against the oracle (oracle/w8a8.py) and
the golden brute force (tests/golden/w8a8.npz).  Everything here is integer work or single
rounded f32 operations, so the bar is bit-exact: int8 operands, int32 accumulators, f32
scales and the bf16 output must all match exactly."""

import os

import numpy as np
import pytest
import torch

from flicker_amd import w8a8, workloads
from oracle import w8a8 as Q
from oracle.numerics import bf16_bits, from_bf16_bits

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def host(t):
    return t.detach().cpu().numpy()


def host_f32(t):
    return t.detach().to("cpu", torch.float32).numpy()


def assert_bits_equal(got_bf16: torch.Tensor, want_f32: np.ndarray, label: str):
    got = bf16_bits(host_f32(got_bf16))
    want = bf16_bits(np.asarray(want_f32, np.float32))
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{label}: {len(bad)} of {got.size} differ, first at {bad[0].tolist()}"


def test_golden_pipeline_bit_exact(device):
    """The brute-force fixture (5 tokens, 16 -> 6 channels, one outlier channel, one zero
    token), zero-padded to the kernels' k % 128 and n % 8: padding adds zero channels, which
    leave every smoothing factor, scale and product of the real channels unchanged."""
    g = np.load(os.path.join(GOLDEN, "w8a8.npz"))
    x = from_bf16_bits(g["x"])
    w = from_bf16_bits(g["w"])
    m, k = x.shape
    n = w.shape[1]
    kp, np_ = 128, 8
    xp = np.zeros((m, kp), np.float32)
    xp[:, :k] = x
    wp = np.zeros((kp, np_), np.float32)
    wp[:k, :n] = w
    xt = torch.from_numpy(xp).to(torch.bfloat16).to(device)
    wt = torch.from_numpy(wp).to(torch.bfloat16).to(device)

    qw = w8a8.quantize_linear(wt, w8a8.absmax_cols(xt))
    np.testing.assert_array_equal(host(qw.smooth)[:k], g["smooth"])
    np.testing.assert_array_equal(host(qw.inv_smooth)[:k], g["inv_smooth"])
    np.testing.assert_array_equal(host(qw.w_scale)[:n], g["w_scale"])
    np.testing.assert_array_equal(host(qw.wq_t)[:n, :k].T, g["wq"])

    xq, a_scale = w8a8.quantize_act(xt, qw.inv_smooth)
    np.testing.assert_array_equal(host(xq)[:, :k], g["xq"])
    np.testing.assert_array_equal(host(a_scale), g["a_scale"])

    acc = torch.empty((m, np_), dtype=torch.int32, device=device)
    y = w8a8.gemm(xq, a_scale, qw.wq_t, qw.w_scale, acc=acc)
    np.testing.assert_array_equal(host(acc)[:, :n], g["acc"])
    np.testing.assert_array_equal(bf16_bits(host_f32(y))[:, :n], g["y"])


def calib_inputs(m=777, k=320, n=264, seed=7):
    """bf16 X with outlier channels, an all-zero channel and an all-zero token; bf16 W with an
    all-zero input row."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=g)
    x[:, 5] *= 30.0
    x[:, 9] = 0.0
    x[3] = 0.0
    w = 0.02 * torch.randn((k, n), generator=g)
    w[11] = 0.0
    return x.to(torch.bfloat16), w.to(torch.bfloat16)


def test_calibration_statistics_and_smoothing(device):
    x, w = calib_inputs()
    xn, wn = x.float().numpy(), w.float().numpy()
    xa = w8a8.absmax_cols(x.to(device))
    wa = w8a8.absmax_rows(w.to(device))
    np.testing.assert_array_equal(host(xa), np.abs(xn).max(0))
    np.testing.assert_array_equal(host(wa), np.abs(wn).max(1))
    # running maximum over two calibration batches equals the maximum over their union
    run = w8a8.absmax_cols(x[:400].to(device))
    w8a8.absmax_cols(x[400:].to(device), out=run)
    np.testing.assert_array_equal(host(run), np.abs(xn).max(0))
    s, inv = w8a8.smooth_factors(xa, wa)
    s_want = Q.smooth_factors(np.abs(xn).max(0), np.abs(wn).max(1))
    np.testing.assert_array_equal(host(s), s_want)
    np.testing.assert_array_equal(host(inv), Q.inverse(s_want))
    assert host(s)[9] == 1.0 and host(s)[11] == 1.0       # zero activation / zero weight row


def test_quantize_weight_full_size_bit_exact(device):
    p = workloads.PROJECTIONS["qkv_1024"]
    x, w = workloads.make_projection(p)
    xa = np.abs(x.float().numpy()).max(0)
    wn = w.float().numpy()
    s = Q.smooth_factors(xa, np.abs(wn).max(1))
    wq_want, ws_want = Q.quantize_weight(wn, s)
    wq_t, ws = w8a8.quantize_weight(w.to(device), torch.from_numpy(s).to(device))
    np.testing.assert_array_equal(host(ws), ws_want)
    np.testing.assert_array_equal(host(wq_t), wq_want.T)


@pytest.mark.parametrize("strided", [False, True])
def test_quantize_act_bit_exact(device, strided):
    p = workloads.PROJECTIONS["qkv_1024"]
    x, _ = workloads.make_projection(p)
    x[17] = 0.0                                                   # zero token: scale 1, all zeros
    inv = Q.inverse(Q.smooth_factors(np.abs(x.float().numpy()).max(0) * 0.5 + 0.25,
                                     np.full(p.hidden, 0.06, np.float32)))
    xd = x.to(device)
    if strided:                                                   # a column block of a wider activation
        wide = torch.zeros((p.tokens, p.hidden + 512), dtype=torch.bfloat16, device=device)
        wide[:, 256:256 + p.hidden] = xd
        xd = wide[:, 256:256 + p.hidden]
    xq, a = w8a8.quantize_act(xd, torch.from_numpy(inv).to(device))
    xq_want, a_want = Q.quantize_act(x.float().numpy(), inv)
    np.testing.assert_array_equal(host(a), a_want)
    np.testing.assert_array_equal(host(xq), xq_want)
    assert host(a)[17] == 1.0


def test_quantize_act_near_ties(device):
    """Rows whose quotients sit next to half-integers (v = amax / 2 -> v / a ~ 63.5), where a
    reciprocal multiply rounds differently from the division: the kernel's fast path must
    hand these to the division.  Each row also holds random values below its amax."""
    from tests.test_oracle_pins import NEAR_TIE_ROWS
    rng = np.random.default_rng(17)
    k = 512
    rows = []
    for amax in NEAR_TIE_ROWS:
        r = rng.uniform(-amax, amax, k).astype(np.float32)
        r[0], r[1], r[2] = amax, amax / 2, -amax / 2
        rows.append(r)
    x = torch.from_numpy(np.stack(rows)).to(torch.bfloat16)
    inv = np.ones(k, np.float32)
    xq, a = w8a8.quantize_act(x.to(device), torch.from_numpy(inv).to(device))
    xq_want, a_want = Q.quantize_act(x.float().numpy(), inv)
    np.testing.assert_array_equal(host(a), a_want)
    np.testing.assert_array_equal(host(xq), xq_want)


@pytest.mark.parametrize("m,k,n", [(300, 256, 520), (1, 128, 4), (257, 3072, 260), (512, 128, 1024),
                                   (4608, 3072, 9216 // 36), (2600, 384, 6000)])
def test_gemm_tails_bit_exact(device, m, k, n):
    """Ragged tiles in both output dimensions; full-range int8 operands.  The last case has
    11 x 24 = 264 tiles, more than one round of 256 CUs: the rounds order runs 256 of them
    whole and cuts the queries of the rest into 192-token tiles, ragged ones included."""
    rng = np.random.default_rng(m * 7 + n)
    xq = rng.integers(-127, 128, (m, k), dtype=np.int8)
    wq = rng.integers(-127, 128, (k, n), dtype=np.int8)
    a = (rng.random(m, dtype=np.float32) * 0.05 + 1e-3).astype(np.float32)
    ws = (rng.random(n, dtype=np.float32) * 0.002 + 1e-5).astype(np.float32)
    acc = torch.empty((m, n), dtype=torch.int32, device=device)
    y = w8a8.gemm(torch.from_numpy(xq).to(device), torch.from_numpy(a).to(device),
                  torch.from_numpy(np.ascontiguousarray(wq.T)).to(device), torch.from_numpy(ws).to(device), acc=acc)
    acc_want = Q.int_gemm(xq, wq)
    np.testing.assert_array_equal(host(acc), acc_want)
    assert_bits_equal(y, Q.rescale(acc_want, a, ws), f"y {m}x{k}x{n}")


@pytest.mark.parametrize("m,n", [(4352, 9216), (3840, 9216), (4100, 9000), (2600, 9216), (6000, 6144),
                                 (4096, 4096), (4097, 4096), (4096, 4100), (8192, 8192), (8193, 8192)])
def test_gemm_rounds_order_bit_exact(device, m, n):
    """Grids of more than one round (the Klein QKV widths): whole rounds of 256 x 256 tiles,
    then the tiles left over cut into 192-token tiles, runs of one channel tile starting and
    ending between token tiles, the last tile of a run cut short; and around the choice: exactly
    one round (256 tiles), one tile row or column more, whole rounds with nothing left over,
    and those plus one row.  Every int32 product and bf16 output against the oracle (K = 128
    keeps the float64 oracle product quick)."""
    k = 128
    rng = np.random.default_rng(m + n)
    xq = rng.integers(-127, 128, (m, k), dtype=np.int8)
    wq = rng.integers(-127, 128, (k, n), dtype=np.int8)
    a = (rng.random(m, dtype=np.float32) * 0.05 + 1e-3).astype(np.float32)
    ws = (rng.random(n, dtype=np.float32) * 0.002 + 1e-5).astype(np.float32)
    acc = torch.empty((m, n), dtype=torch.int32, device=device)
    y = w8a8.gemm(torch.from_numpy(xq).to(device), torch.from_numpy(a).to(device),
                  torch.from_numpy(np.ascontiguousarray(wq.T)).to(device), torch.from_numpy(ws).to(device), acc=acc)
    acc_want = Q.int_gemm(xq, wq)
    np.testing.assert_array_equal(host(acc), acc_want)
    assert_bits_equal(y, Q.rescale(acc_want, a, ws), f"y {m}x{k}x{n}")


def test_gemm_random_shapes_bit_exact(device):
    """Seeded random projections around one round of tiles (some take the rounds order, some
    the plain order, ragged edges in both dimensions): every int32 product and bf16 output
    against the oracle."""
    rng = np.random.default_rng(77)
    for trial in range(6):
        while True:
            m, n = int(rng.integers(1, 9000)), 4 * int(rng.integers(1, 3000))
            if 200 <= -(-m // 256) * -(-n // 256) <= 700:
                break
        k = 128 * int(rng.integers(1, 3))
        xq = rng.integers(-127, 128, (m, k), dtype=np.int8)
        wq = rng.integers(-127, 128, (k, n), dtype=np.int8)
        a = (rng.random(m, dtype=np.float32) * 0.05 + 1e-3).astype(np.float32)
        ws = (rng.random(n, dtype=np.float32) * 0.002 + 1e-5).astype(np.float32)
        acc = torch.empty((m, n), dtype=torch.int32, device=device)
        y = w8a8.gemm(torch.from_numpy(xq).to(device), torch.from_numpy(a).to(device),
                      torch.from_numpy(np.ascontiguousarray(wq.T)).to(device), torch.from_numpy(ws).to(device),
                      acc=acc)
        acc_want = Q.int_gemm(xq, wq)
        np.testing.assert_array_equal(host(acc), acc_want, err_msg=f"{m}x{k}x{n}")
        assert_bits_equal(y, Q.rescale(acc_want, a, ws), f"y {m}x{k}x{n}")


def test_gemm_extreme_operands(device):
    """All operands at +-127: the largest |acc| the int32 accumulator sees at K = 3072."""
    m, k, n = 64, 3072, 64
    xq = np.full((m, k), 127, np.int8)
    xq[1::2] = -127
    wq = np.full((k, n), 127, np.int8)
    acc = torch.empty((m, n), dtype=torch.int32, device=device)
    w8a8.gemm(torch.from_numpy(xq).to(device), torch.ones(m, device=device),
              torch.from_numpy(np.ascontiguousarray(wq.T)).to(device), torch.ones(n, device=device), acc=acc)
    got = host(acc)
    assert got[0, 0] == 3072 * 127 * 127 and got[1, 0] == -3072 * 127 * 127
    np.testing.assert_array_equal(got, Q.int_gemm(xq, wq))


def test_projection_full_size_bit_exact(device):
    """The 1024^2 Klein QKV projection (4608 x 3072 -> 9216): calibrate on the input itself,
    quantise, multiply; every int32 product and every bf16 output against the oracle."""
    p = workloads.PROJECTIONS["qkv_1024"]
    x, w = workloads.make_projection(p)
    xd, wd = x.to(device), w.to(device)
    qw = w8a8.quantize_linear(wd, w8a8.absmax_cols(xd))
    xq, a = w8a8.quantize_act(xd, qw.inv_smooth)
    acc = torch.empty((p.tokens, p.out_features), dtype=torch.int32, device=device)
    y = w8a8.gemm(xq, a, qw.wq_t, qw.w_scale, acc=acc)

    xn, wn = x.float().numpy(), w.float().numpy()
    s = Q.smooth_factors(np.abs(xn).max(0), np.abs(wn).max(1))
    wq_want, ws_want = Q.quantize_weight(wn, s)
    y_want, acc_want, xq_want, a_want = Q.w8a8_linear(xn, Q.inverse(s), wq_want, ws_want)
    np.testing.assert_array_equal(host(xq), xq_want)
    np.testing.assert_array_equal(host(a), a_want)
    np.testing.assert_array_equal(host(acc), acc_want)
    assert_bits_equal(y, y_want, "y full projection")
    # and the fused path (no acc written) gives the same output
    y2 = w8a8.linear(xd, qw)
    assert torch.equal(y2, y)


def test_linear_writes_into_strided_output(device):
    """Y written straight into the qkv columns of a wider (linear1-style) buffer."""
    x, w = calib_inputs(m=130, k=256, n=384)
    xd, wd = x.to(device), w.to(device)
    qw = w8a8.quantize_linear(wd, w8a8.absmax_cols(xd))
    wide = torch.full((130, 384 + 128), 7.0, dtype=torch.bfloat16, device=device)
    w8a8.linear(xd, qw, out=wide[:, :384])
    assert torch.equal(wide[:, :384], w8a8.linear(xd, qw))
    assert bool((wide[:, 384:] == 7.0).all())


def test_quantisation_error_against_bf16_projection(device):
    """Sanity of the int8 replacement against the bf16 projection it stands in for
    (nn.py:13-14): relative Frobenius error of a few percent on outlier-heavy activations."""
    p = workloads.PROJECTIONS["qkv_512"]
    x, w = workloads.make_projection(p)
    xd, wd = x.to(device), w.to(device)
    y = w8a8.linear(xd, w8a8.quantize_linear(wd, w8a8.absmax_cols(xd)))
    ref = x.double().numpy() @ w.double().numpy()
    rel = np.linalg.norm(host_f32(y) - ref) / np.linalg.norm(ref)
    assert rel < 0.03, rel


def _fused_case(device, batch, length, heads, k, scale_dtype, gain, seed):
    from flicker_amd import kernels, rope
    from oracle import path as P
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, length, k, generator=g)
    x[..., 5] *= 20.0                                                # an outlier channel
    w = 0.02 * torch.randn(k, 3 * heads * 128, generator=g)
    qs = (1 + 0.05 * torch.randn(128, generator=g)).to(scale_dtype)
    ks = (1 + 0.05 * torch.randn(128, generator=g)).to(scale_dtype)
    x, w = x.to(torch.bfloat16).to(device), w.to(torch.bfloat16).to(device)
    qw = w8a8.quantize_linear(w, w8a8.absmax_cols(x))
    ids = P.sequence_ids(min(length, 16), 1, max(length - 16, 0)) if length > 16 else P.sequence_ids(length, 0, 0)
    freqs = rope.rope_lanes(ids, gain, device=device)
    qs, ks = qs.to(device), ks.to(device)
    return x, qw, qs, ks, freqs, kernels


@pytest.mark.parametrize("batch,length,heads,k,scale_dtype,gain", [
    (1, 4608, 24, 3072, torch.bfloat16, 128 ** -0.5),   # the 1024^2 Klein projection feeding qk_prep
    (2, 257, 2, 256, torch.float32, 1.0),               # ragged token tiles, f32 scales, no gain
    (1, 40, 3, 128, torch.bfloat16, 0.3),
    (7, 3, 2, 128, torch.bfloat16, 0.5),                # sequences shorter than a read-back step
    (5, 67, 2, 128, torch.bfloat16, 128 ** -0.5),       # batch entries wrapping inside every tile
    (2, 2176, 24, 128, torch.float32, 128 ** -0.5),     # rounds order, batch entries wrapping in 192-token tiles
    (3, 1300, 24, 128, torch.bfloat16, 0.5),            # rounds order, ragged last token tile
])
def test_fused_projection_qk_prep_bit_exact(device, batch, length, heads, k, scale_dtype, gain):
    """flk_w8a8_qk_prep == flk_qk_prep(flk_w8a8_gemm(...)) bit for bit: the epilogue applies
    the same row arithmetic (one shared implementation) to the same bf16 projected values."""
    x, qw, qs, ks, freqs, kernels = _fused_case(device, batch, length, heads, k, scale_dtype, gain, seed=length)
    y = w8a8.linear(x, qw)
    want = kernels.qk_prep(y, qs, ks, freqs, heads, rows=length)
    got = w8a8.qk_prep(x, qw, qs, ks, freqs, heads)
    torch.cuda.synchronize()
    for name, a, b in zip("qkv", got, want):
        assert a.shape == b.shape == (batch, heads, length, 128)
        bad = int((a.view(torch.int16) != b.view(torch.int16)).sum())
        assert bad == 0, f"{name}: {bad} of {a.numel()} elements differ"


def test_fused_projection_random_shapes_bit_exact(device):
    """Seeded random projections feeding qk_prep (batches whose entries wrap inside token
    tiles, ragged lengths, 1-24 heads, k up to 384, both scale types, gains; alternately
    within and past one round of tiles), each equal to the GEMM followed by qk_prep, bit
    for bit."""
    rng = np.random.default_rng(91)
    for trial in range(6):
        while True:   # odd trials past one round of 256 x 256 tiles (the rounds order)
            batch, length = int(rng.integers(1, 5)), int(rng.integers(1, 3000))
            heads, k = int(rng.integers(1, 25)), 128 * int(rng.integers(1, 4))
            tiles = -(-batch * length // 256) * -(-3 * heads * 128 // 256)
            if (256 < tiles <= 700) if trial % 2 else (tiles <= 256):
                break
        scale_dtype = torch.float32 if trial % 2 else torch.bfloat16
        gain = float(rng.choice([1.0, 128 ** -0.5, 0.3]))
        label = f"B{batch} L{length} H{heads} k{k} {scale_dtype} gain{gain:.4f}"
        print(label, flush=True)
        x, qw, qs, ks, freqs, kernels = _fused_case(device, batch, length, heads, k, scale_dtype, gain,
                                                    seed=900 + trial)
        want = kernels.qk_prep(w8a8.linear(x, qw), qs, ks, freqs, heads, rows=length)
        got = w8a8.qk_prep(x, qw, qs, ks, freqs, heads)
        torch.cuda.synchronize()
        for name, a, b in zip("qkv", got, want):
            bad = int((a.view(torch.int16) != b.view(torch.int16)).sum())
            assert bad == 0, f"{label} {name}: {bad} of {a.numel()} elements differ"


def test_fused_projection_accepts_position_ids(device):
    """w8a8.qk_prep with PositionIds equals the table form (the lanes are built from the ids)."""
    from flicker_amd import rope
    x, qw, qs, ks, freqs, kernels = _fused_case(device, 1, 96, 2, 256, torch.bfloat16, 0.25, seed=3)
    ids = torch.from_numpy(rope.sequence_ids(32, 8, 8)).to(device)
    tables = w8a8.qk_prep(x, qw, qs, ks, rope.rope_lanes(ids, 0.25), 2)
    from_ids = w8a8.qk_prep(x, qw, qs, ks, rope.position_ids(ids, 0.25), 2)
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(tables, from_ids))


def test_fused_projection_writes_at_sequence_offset(device):
    """out/out_offset place the stream inside a joint text|image buffer, as for qk_prep."""
    x, qw, qs, ks, freqs, kernels = _fused_case(device, 1, 64, 2, 128, torch.bfloat16, 0.5, seed=3)
    joint = tuple(torch.full((1, 2, 100, 128), 3.0, dtype=torch.bfloat16, device=device) for _ in range(3))
    w8a8.qk_prep(x, qw, qs, ks, freqs, 2, out=joint, out_offset=20)
    want = kernels.qk_prep(w8a8.linear(x, qw), qs, ks, freqs, 2)
    torch.cuda.synchronize()
    for a, b in zip(joint, want):
        assert torch.equal(a[:, :, 20:84].view(torch.int16), b.view(torch.int16))
        assert bool((a[:, :, :20] == 3.0).all()) and bool((a[:, :, 84:] == 3.0).all())


@pytest.mark.parametrize("batch,length,k", [(2, 300, 3072), (1, 5, 200), (3, 17, 512)])
def test_modulated_activation_bit_exact(device, batch, length, k):
    """flk_quantize_act_modulated: X = modulate(x) (modules.py:38-40) equals the oracle bit for
    bit (f64 row statistics make the mean order-free), and its int8 quantisation equals both
    the oracle's and the unfused quantize_act of that X."""
    g = torch.Generator().manual_seed(k + length)
    x = 2.0 * torch.randn(batch, length, k, generator=g) + 0.3
    x[..., 7] *= 15.0                                                 # an outlier channel
    shift = 0.5 * torch.randn(batch, k, generator=g)
    scale = 0.2 * torch.randn(batch, k, generator=g)
    x, shift, scale = (t.to(torch.bfloat16) for t in (x, shift, scale))
    inv_s = (0.5 + torch.rand(k, generator=g)).to(device)
    xq, a_scale, x_mod = w8a8.quantize_act_modulated(x.to(device), shift.to(device), scale.to(device), inv_s,
                                                     x_mod=True)
    want_mod = Q.modulate(host_f32(x), host_f32(shift), host_f32(scale))
    assert_bits_equal(x_mod, want_mod, "modulated X")
    want_q, want_a = Q.quantize_act(want_mod.reshape(-1, k), host(inv_s))
    np.testing.assert_array_equal(host(xq), want_q)
    np.testing.assert_array_equal(host(a_scale), want_a)
    xq2, a2 = w8a8.quantize_act(x_mod, inv_s)
    assert torch.equal(xq2, xq) and torch.equal(a2, a_scale)


def test_modulated_projection_qk_prep(device):
    """The whole qkv_prep(linear(modulate(x, mod1), w), ...) of a block in two launches equals
    the step-by-step path (modulated X, then the fused projection + qk_prep)."""
    x, qw, qs, ks, freqs, kernels = _fused_case(device, 1, 300, 3, 256, torch.bfloat16, 0.3, seed=21)
    g = torch.Generator().manual_seed(22)
    shift = (0.3 * torch.randn(1, 256, generator=g)).to(torch.bfloat16).to(device)
    scale = (0.1 * torch.randn(1, 256, generator=g)).to(torch.bfloat16).to(device)
    got = w8a8.qk_prep(x, qw, qs, ks, freqs, 3, modulation=(shift, scale))
    _, _, x_mod = w8a8.quantize_act_modulated(x, shift, scale, qw.inv_smooth, x_mod=True)
    want = w8a8.qk_prep(x_mod, qw, qs, ks, freqs, 3)
    torch.cuda.synchronize()
    for a, b in zip(got, want):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("batch,len0,len1,heads,k,scale_dtype,modulated", [
    (1, 512, 4096, 24, 3072, torch.bfloat16, False),   # a Klein double block: 512 text + 64x64 image tokens
    (2, 70, 300, 2, 256, torch.float32, True),          # ragged streams, f32 scales, modulated inputs
    (1, 0, 130, 2, 128, torch.bfloat16, False),         # an empty text stream
])
def test_fused_projection_pair_equals_two_calls(device, batch, len0, len1, heads, k, scale_dtype, modulated):
    """flk_w8a8_qk_prep_pair (both streams of a double block in one launch) writes exactly what
    two flk_w8a8_qk_prep calls write at sequence offsets 0 and L_txt: each stream has its own
    weights, norm scales, RoPE rows and (optionally) modulation."""
    from flicker_amd.kernels import Freqs
    gain = 128 ** -0.5
    streams, mods = [], []
    for i, n in enumerate((len0, len1)):
        x, qw, qs, ks, freqs, _ = _fused_case(device, batch, max(n, 1), heads, k, scale_dtype, gain, seed=40 + i)
        streams.append((x[:, :n].contiguous(), qw, qs, ks, Freqs(freqs.cos[:n], freqs.sin[:n], freqs.q_gain)))
        g = torch.Generator().manual_seed(50 + i)
        mods.append(((0.3 * torch.randn(batch, k, generator=g)).to(torch.bfloat16).to(device),
                     (0.1 * torch.randn(batch, k, generator=g)).to(torch.bfloat16).to(device)))
    mods = mods if modulated else [None, None]
    want = tuple(torch.full((batch, heads, len0 + len1, 128), 5.0, dtype=torch.bfloat16, device=device)
                 for _ in range(3))
    w8a8.qk_prep(*streams[0], heads, out=want, out_offset=0, modulation=mods[0])
    w8a8.qk_prep(*streams[1], heads, out=want, out_offset=len0, modulation=mods[1])
    got = w8a8.qk_prep_pair(streams[0], streams[1], heads, modulation=(mods[0], mods[1]) if modulated else None)
    torch.cuda.synchronize()
    for name, a, b in zip("qkv", got, want):
        bad = int((a.view(torch.int16) != b.view(torch.int16)).sum())
        assert bad == 0, f"{name}: {bad} of {a.numel()} elements differ"


@pytest.mark.parametrize("batch,len0,len1,k", [(1, 512, 4096, 3072), (2, 7, 130, 200), (1, 0, 33, 256)])
def test_modulated_activation_pair_equals_two_calls(device, batch, len0, len1, k):
    """flk_quantize_act_modulated_pair: both streams' codes and scales equal their own
    flk_quantize_act_modulated bit for bit (an empty text stream included)."""
    g = torch.Generator().manual_seed(k + len1)
    out = []
    for n in (len0, len1):
        x = (2.0 * torch.randn(batch, n, k, generator=g) + 0.3).to(torch.bfloat16).to(device)
        shift = (0.5 * torch.randn(batch, k, generator=g)).to(torch.bfloat16).to(device)
        scale = (0.2 * torch.randn(batch, k, generator=g)).to(torch.bfloat16).to(device)
        inv_s = (0.5 + torch.rand(k, generator=g)).to(device)
        out.append((x, shift, scale, inv_s))
    got = w8a8.quantize_act_modulated_pair(*out[0], *out[1])
    for (xq, a_scale), args in zip(got, out):
        want_q, want_a = w8a8.quantize_act_modulated(*args)
        torch.cuda.synchronize()
        assert torch.equal(xq, want_q) and torch.equal(a_scale, want_a)
    with pytest.raises(ValueError, match="one width"):
        x_other = torch.zeros(batch, 4, k + 8, dtype=torch.bfloat16, device=device)
        w8a8.quantize_act_modulated_pair(*out[0], x_other, out[1][1][:, :1].expand(batch, k + 8).contiguous(),
                                         out[1][2][:, :1].expand(batch, k + 8).contiguous(),
                                         torch.ones(k + 8, device=device))


def test_errors(device):
    x = torch.zeros((4, 100), dtype=torch.bfloat16, device=device)
    with pytest.raises(Exception, match="status -3"):        # k % 8
        w8a8.quantize_act(x[:, :98], torch.ones(98, device=device))
    xq = torch.zeros((4, 96), dtype=torch.int8, device=device)
    with pytest.raises(Exception, match="status -3"):        # k % 128
        w8a8.gemm(xq, torch.ones(4, device=device), torch.zeros((8, 96), dtype=torch.int8, device=device),
                  torch.ones(8, device=device))
    with pytest.raises(ValueError, match="input channels"):
        w8a8.gemm(xq, torch.ones(4, device=device), torch.zeros((8, 64), dtype=torch.int8, device=device),
                  torch.ones(8, device=device))
    with pytest.raises(ValueError, match="GPU"):
        w8a8.quantize_act(torch.zeros((4, 64), dtype=torch.bfloat16), torch.ones(64))


def test_double_attention_int8_equals_step_by_step(device):
    """modules.double_attention_int8 (paired quantisation, paired projection + qk_prep, one
    joint attention) equals the int8 path run stream by stream into the joint buffer."""
    from flicker_amd import kernels, modules
    from flicker_amd.kernels import Freqs
    heads, k, n_txt, n_img = 2, 256, 40, 200
    txt_x, txt_qw, qs0, ks0, f0, _ = _fused_case(device, 1, n_txt, heads, k, torch.bfloat16, 0.25, seed=61)
    img_x, img_qw, qs1, ks1, _, _ = _fused_case(device, 1, n_img, heads, k, torch.bfloat16, 0.25, seed=62)
    from flicker_amd import rope
    from oracle import path as P
    freqs = rope.rope_lanes(P.sequence_ids(n_txt, 10, 20), 0.25, device=device)
    g = torch.Generator().manual_seed(63)
    mods = tuple(((0.3 * torch.randn(1, k, generator=g)).to(torch.bfloat16).to(device),
                  (0.1 * torch.randn(1, k, generator=g)).to(torch.bfloat16).to(device)) for _ in range(2))
    got_txt, got_img = modules.double_attention_int8(txt_x, img_x, txt_qw, img_qw, (qs0, ks0), (qs1, ks1), freqs,
                                                     heads, modulation=mods)
    joint = tuple(torch.empty(1, heads, n_txt + n_img, 128, dtype=torch.bfloat16, device=device) for _ in range(3))
    cut = lambda a, b: Freqs(freqs.cos[a:b], freqs.sin[a:b], freqs.q_gain)  # noqa: E731
    w8a8.qk_prep(txt_x, txt_qw, qs0, ks0, cut(0, n_txt), heads, out=joint, out_offset=0, modulation=mods[0])
    w8a8.qk_prep(img_x, img_qw, qs1, ks1, cut(n_txt, n_txt + n_img), heads, out=joint, out_offset=n_txt,
                 modulation=mods[1])
    want = kernels.attend_merged(*joint)
    torch.cuda.synchronize()
    assert torch.equal(got_txt, want[:, :n_txt]) and torch.equal(got_img, want[:, n_txt:])
