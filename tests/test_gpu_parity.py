"""GPU parity: the HIP kernels, called through the C ABI, against the CPU oracle.

Bars (stated per test):
  * quantize / dequantize: bit-exact (integer and bf16-bit work);
  * qmatmul: within half a bf16 ulp of the fp64 reference plus 2^-18 * max|ref| (the
    GEMV against exact dequantization, the MFMA GEMM against its bf16 weights), and
    sig_rel = max|d|/max|ref| <= 1e-2 against the fp64 ground truth;
  * exact-arithmetic inputs (x in {-1,0,1}, scale 2^-7): bit-exact;
  * fused gelu/softcap epilogues: bit-exact against the oracle applied to the
    kernel's own matmul outputs, allowing a 1-ulp difference on at most 0.1% of
    elements where device tanhf and glibc tanhf round differently.
"""
import ctypes
import sys

import numpy as np
import pytest

import hyperion_amd as hy
import oracle as O
import st_reader
from hyperion_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def ulp_diff(a_bits, b_bits):
    """Distance in bf16 ulps between two bf16 bit arrays (same sign assumed near 0)."""
    def key(h):
        h = h.astype(np.int32)
        return np.where(h & 0x8000, -(h & 0x7FFF), h)
    return np.abs(key(a_bits) - key(b_bits))


def assert_within_bf16_rounding(y_bits, truth, what, slack=2.0**-18):
    """|y - truth| <= half a bf16 ulp of truth + slack * max|truth|: the bf16 output
    rounding plus an fp32-accumulation allowance (which is relative to the size of the
    summed terms, so near-zero outputs may be several ulps off in relative terms)."""
    t = np.asarray(truth, np.float64)
    y = syn.bf16_to_f32(y_bits).astype(np.float64)
    tb = syn.bf16_to_f32(syn.bf16_bits(t.astype(np.float32))).astype(np.float64)
    half_ulp = np.abs(tb) * 2.0**-8 + 1e-40            # bf16: 8 significant bits
    bound = half_ulp + slack * float(np.max(np.abs(t)))
    worst = float(np.max(np.abs(y - t) / bound))
    assert worst <= 1.0, f"{what}: worst error {worst:.2f}x the bf16-rounding bound"


def dev(a, stream):
    return hy.DeviceArray.from_host(a, stream)


def run_qmatmul(w, s, b, x, stream, softcap=None):
    qw = hy.QWeight.from_host(w, s, b)
    m, k = x.shape
    n = w.shape[0]
    xd = dev(x, stream)
    yd = hy.DeviceArray((m, n), np.uint16)
    hy.qmatmul(qw, xd, m, yd, stream, softcap=softcap)
    y = yd.to_host(stream)
    qw.close()
    return y


def test_runtime_is_gfx950():
    info = hy.runtime_info()
    say(f"device {info.device_name.decode()} arch {info.arch_name.decode()} CUs {info.compute_units} "
        f"HBM {info.hbm_bytes / 2**30:.0f} GiB")
    assert info.arch_name.decode().startswith("gfx950")
    assert info.abi_version == 1


# ---------------------------------------------------------------- quantize / dequantize

def _gpu_quantize(wbf, stream):
    n, k = wbf.shape
    wd = dev(wbf, stream)
    wq = hy.DeviceArray((n, k // 8), np.uint32)
    sd = hy.DeviceArray((n, k // 64), np.uint16)
    bd = hy.DeviceArray((n, k // 64), np.uint16)
    hy.quantize(wd, n, k, wq, sd, bd, stream)
    return wq.to_host(stream), sd.to_host(stream), bd.to_host(stream)


def test_quantize_pack_config_bit_exact(stream):
    """Quantize/pack workload: bf16 [15360, 3840] N(0, 0.02^2) with 1% x8 outliers."""
    n, k = 15360, 3840
    say(f"quantize n={n} k={k}")
    wbf = syn.quantize_input(n, k, seed=101)
    got = _gpu_quantize(wbf, stream)
    ref = O.quantize(wbf)
    for g, r, name in zip(got, ref, ("packed", "scales", "biases")):
        bad = np.count_nonzero(g != r)
        assert bad == 0, f"{name}: {bad} mismatches"


def test_quantize_reproduces_reference_fixture(stream, fixture_dir):
    """GPU requantization of the fixture's dequantized weights returns MLX's own
    (codes, scale, bias) on every group holding code 15, and equals the oracle on all."""
    total = exact = 0
    for name, (w, s, b) in st_reader.q4_tensors(fixture_dir).items():
        wd = O.dequantize(w, s, b)
        gw, gs, gb = _gpu_quantize(wd, stream)
        ow, os_, ob = O.quantize(wd)
        assert np.array_equal(gw, ow) and np.array_equal(gs, os_) and np.array_equal(gb, ob), name
        codes = syn.unpack_codes(w).reshape(w.shape[0], -1, 64)
        gcodes = syn.unpack_codes(gw).reshape(w.shape[0], -1, 64)
        has15 = (codes == 15).any(-1)
        same = (codes == gcodes).all(-1) & (s == gs) & (b == gb)
        total += int(has15.sum())
        exact += int((same & has15).sum())
    assert total == 16578 and exact == total


def test_quantize_edge_groups(stream):
    """Zero, constant, negative-only, tie-heavy, huge/tiny-magnitude and subnormal groups."""
    rng = np.random.default_rng(5)
    groups = []
    c = np.tile(np.arange(16), 4).astype(np.float64)
    groups.append(np.zeros(64))
    groups.append(np.full(64, 0.01))
    groups.append(np.full(64, -0.25))
    groups.append((c - 8) * 2.0**-7)
    half = c.copy(); half[::3] += 0.5
    groups.append((half - 8) * 2.0**-7)                    # exact .5 quotients
    groups.append(-np.abs(rng.standard_normal(64)) * 0.01)  # all negative
    groups.append(np.abs(rng.standard_normal(64)) * 0.01)   # all positive
    g = rng.standard_normal(64); g[7] = -g.max()            # |min| == |max|
    groups.append(g)
    groups.append(rng.standard_normal(64) * 1e30)
    groups.append(rng.standard_normal(64) * 1e-30)
    groups.append(rng.standard_normal(64) * 1e-39)          # bf16 subnormals
    for _ in range(53):
        groups.append(rng.standard_normal(64) * 10.0 ** rng.uniform(-4, 2))
    w = syn.bf16_bits(np.stack(groups).astype(np.float32).reshape(8, -1))
    got = _gpu_quantize(w, stream)
    ref = O.quantize(w)
    for gv, rv, name in zip(got, ref, ("packed", "scales", "biases")):
        assert np.array_equal(gv, rv), name


@pytest.mark.parametrize("n,k", [(1, 64), (3, 640), (7, 64 * 37), (5, 64 * 52), (257, 128)])
def test_quantize_ragged_group_counts(stream, n, k):
    """Group counts that leave a wave (64 groups) or a workgroup (256) partly empty."""
    say(f"quantize ragged n={n} k={k}")
    w = syn.quantize_input(n, k, seed=n * 1000 + k)
    got = _gpu_quantize(w, stream)
    for gv, rv, name in zip(got, O.quantize(w), ("packed", "scales", "biases")):
        np.testing.assert_array_equal(gv, rv, err_msg=name)


def test_quantize_rejects_misaligned_buffers(stream):
    n, k = 2, 128
    wd = dev(syn.quantize_input(n, k, seed=3), stream)
    wq = hy.DeviceArray((n, k // 8 + 4), np.uint32)
    sd = hy.DeviceArray((n, k // 64 + 1), np.uint16)
    bd = hy.DeviceArray((n, k // 64 + 1), np.uint16)
    shifted = lambda a, by: ctypes.c_void_p(a.ptr.value + by)  # noqa: E731
    for args in ((shifted(wd, 2), wq.ptr), (wd.ptr, shifted(wq, 4))):
        with pytest.raises(hy.HypError) as e:
            hy.call("hyp_quantize_q4g64", args[0], n, k, args[1], sd.ptr, bd.ptr, stream.handle)
        assert e.value.status_name == "INVALID_ARGUMENT" and "aligned" in str(e.value)
    for a in (wd, wq, sd, bd):
        a.close()


def test_dequantize_table_bit_exact(stream):
    n, k = 15360, 3840
    say(f"dequantize n={n} k={k}")
    w, s, b = syn.q4_weights(n, k, seed=102)
    wd, sd, bd = dev(w, stream), dev(s, stream), dev(b, stream)
    out = hy.DeviceArray((n, k), np.uint16)
    hy.dequantize(wd, sd, bd, n, k, None, n, out, stream)
    got = out.to_host(stream)
    ref = O.dequantize(w, s, b)
    assert np.count_nonzero(got != ref) == 0


def test_dequantize_gather_scale_and_out_of_range(stream):
    n, k = 1000, 512
    w, s, b = syn.q4_weights(n, k, seed=103)
    ids = np.array([5, 999, 0, 5, 1000, 123456, 77], np.uint32)
    wd, sd, bd = dev(w, stream), dev(s, stream), dev(b, stream)
    idd = dev(ids, stream)
    out = hy.DeviceArray((ids.size, k), np.uint16)
    hy.dequantize(wd, sd, bd, n, k, idd, ids.size, out, stream, out_scale=float(np.sqrt(k)))
    got = out.to_host(stream)
    valid = ids < n
    ref = O.scale(O.dequantize(w, s, b, rows=ids[valid]), float(np.sqrt(np.float32(k))))
    np.testing.assert_array_equal(got[valid], ref)
    assert np.all(got[~valid] == 0)


def test_embed_reproduces_the_reference_12b_golden(stream):
    """hyp_embed and hyp_dequantize_q4g64 return the bits of the reference's own 12B embed
    golden (forward_12b_test.cc:218) from the Q4 rows recovered from it (tests/embed_fit.py):
    MLX's single-rounded dequantize times bf16(sqrt(3840)), bit for bit."""
    import embed_fit
    _, e = embed_fit.load()
    w, s, b = embed_fit.fitted_rows(e)
    n, k = w.shape[0], w.shape[1] * 8
    ids = np.array([3, 0, 9, 1, 2, 4, 5, 6, 7, 8], np.uint32)
    say(f"12B embed golden: {n} rows k={k}")
    qw = hy.QWeight.from_host(w, s, b)
    out = hy.DeviceArray((ids.size, k), np.uint16)
    hy.embed(qw, dev(ids, stream), ids.size, out, stream)
    np.testing.assert_array_equal(out.to_host(stream), e[ids])
    qw.close()
    wd, sd, bd = dev(w, stream), dev(s, stream), dev(b, stream)
    out2 = hy.DeviceArray((n, k), np.uint16)
    hy.dequantize(wd, sd, bd, n, k, None, n, out2, stream, out_scale=float(np.sqrt(np.float32(k))))
    np.testing.assert_array_equal(out2.to_host(stream), e)


# ---------------------------------------------------------------- decode GEMV

def test_gemv_decode_config(stream):
    """Decode GEMV: x [1,3840] N(0,1), W [15360,3840] Q4/g64 (scale |N|*0.02/7.5, bias -8*scale)."""
    n, k = 15360, 3840
    say(f"gemv m=1 n={n} k={k}")
    x = syn.activations(1, k, seed=104)
    w, s, b = syn.q4_weights(n, k, seed=105)
    y = run_qmatmul(w, s, b, x, stream)
    truth = O.qmatmul_f64(x, w, s, b)
    rel = syn.sig_rel(syn.bf16_to_f32(y), truth)
    mlx_rows = 2048
    mlx = syn.bf16_to_f32(O.qmatmul_mlx_cpu(x, w, s, b, rows=(0, mlx_rows)))
    ref_rel = syn.sig_rel(mlx, truth[:, :mlx_rows])
    say(f"  sig_rel gpu={rel:.3e}  mlx-cpu restatement={ref_rel:.3e} (first {mlx_rows} rows)")
    assert rel <= 1e-2
    assert_within_bf16_rounding(y, truth, "decode")


def test_gemv_exact_integer_inputs(stream):
    rng = np.random.default_rng(7)
    for m, n, k in ((1, 512, 3840), (4, 300, 4096), (3, 64, 15360), (2, 33, 128)):
        x = rng.integers(-1, 2, size=(m, k)).astype(np.float32)
        codes = rng.integers(0, 16, size=(n, k)).astype(np.uint8)
        w = syn.pack_codes(codes)
        s = syn.bf16_bits(np.full((n, k // 64), 2.0**-7, np.float32))
        b = syn.bf16_bits(np.full((n, k // 64), -(2.0**-4), np.float32))
        exact = (x.astype(np.int64) @ (codes.astype(np.int64) - 8).T) * 2.0**-7
        y = run_qmatmul(w, s, b, syn.bf16_bits(x), stream)
        np.testing.assert_array_equal(y, syn.bf16_bits(exact.astype(np.float32)), err_msg=f"{m}x{n}x{k}")


def test_gemv_one_hot_pins_layout(stream):
    n, k = 96, 4096
    w, s, b = syn.q4_weights(n, k, seed=106)
    deq = O.dequantize(w, s, b, mode=1)
    for j in (0, 1, 7, 8, 31, 32, 63, 64, 2047, 2048, 4095):
        x = np.zeros((1, k), np.float32)
        x[0, j] = 1.0
        y = run_qmatmul(w, s, b, syn.bf16_bits(x), stream)
        np.testing.assert_array_equal(y[0], deq[:, j], err_msg=f"column {j}")


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_gemv_layer_projections(stream, m):
    """The decoder-layer projection set at decode batch m (split-K path for down)."""
    for i, (name, (n, k)) in enumerate(syn.LAYER_SHAPES.items()):
        say(f"gemv m={m} {name} n={n} k={k}")
        x = syn.activations(m, k, seed=200 + i)
        w, s, b = syn.q4_weights(n, k, seed=300 + i)
        y = run_qmatmul(w, s, b, x, stream)
        truth = O.qmatmul_f64(x, w, s, b)
        assert syn.sig_rel(syn.bf16_to_f32(y), truth) <= 1e-2, name
        assert_within_bf16_rounding(y, truth, name)


def run_group(ws, x, stream):
    """hyp_qmatmul_group over the weights (MLX tensors) -> list of host outputs."""
    qws = [hy.QWeight.from_host(*w) for w in ws]
    m = x.shape[0]
    xd = dev(x, stream)
    yds = [hy.DeviceArray((m, w[0].shape[0]), np.uint16) for w in ws]
    hy.qmatmul_group(qws, xd, m, yds, stream)
    ys = [yd.to_host(stream) for yd in yds]
    for q in qws:
        q.close()
    return ys


@pytest.mark.parametrize("m", [1, 4, 5])
def test_qmatmul_group_qkv(stream, m):
    """q, k and v of one attention block in one grouped call (one launch at m <= 4,
    the GEMM per weight above): each output meets the same bars as hyp_qmatmul."""
    k = 3840
    ws = [syn.q4_weights(n, k, seed=1200 + i) for i, n in enumerate((4096, 2048, 2048))]
    x = syn.activations(m, k, seed=1210 + m)
    ys = run_group(ws, x, stream)
    for (w, s, b), y, name in zip(ws, ys, ("q", "k", "v")):
        say(f"group m={m} {name}")
        if m <= 4:
            truth = O.qmatmul_f64(x, w, s, b)
        else:
            truth = O.qmatmul_deq_f64(x, w, s, b, mode=1)
        assert syn.sig_rel(syn.bf16_to_f32(y), truth) <= 1e-2, name
        assert_within_bf16_rounding(y, truth, name)


def test_qmatmul_group_ragged_segments(stream):
    """Segments of 3, 2 and 1 row tiles (n = 40, 24, 8, partly empty last tiles) and an
    odd group count: workgroups straddle segment boundaries; every output matches the
    fp64 reference, and nothing is written past a segment's n."""
    k = 192
    ws = [syn.q4_weights(n, k, seed=1220 + n) for n in (40, 24, 8)]
    for m in (1, 2, 3, 4):
        say(f"ragged group m={m}")
        x = syn.activations(m, k, seed=1230 + m)
        qws = [hy.QWeight.from_host(*w) for w in ws]
        xd = dev(x, stream)
        # One buffer with a guard band after each output: the kernel must not touch it.
        sentinel = np.full((m * 64,), 0x7FC1, np.uint16)
        yds = []
        for w in ws:
            buf = np.concatenate([np.zeros(m * w[0].shape[0], np.uint16), sentinel])
            yds.append(dev(buf, stream))
        hy.qmatmul_group(qws, xd, m, yds, stream)   # outputs start at each buffer's base
        for (w, s, b), yd in zip(ws, yds):
            n = w.shape[0]
            got = yd.to_host(stream)
            assert np.array_equal(got[m * n:], sentinel), f"n={n}: write past the output"
            assert_within_bf16_rounding(got[:m * n].reshape(m, n), O.qmatmul_f64(x, w, s, b), f"n={n} m={m}")
        for q in qws:
            q.close()


def test_qmatmul_group_rejects_mixed_k(stream):
    a = hy.QWeight.from_host(*syn.q4_weights(16, 128, seed=1240))
    b = hy.QWeight.from_host(*syn.q4_weights(16, 192, seed=1241))
    x = dev(syn.activations(1, 128, seed=1242), stream)
    ys = [hy.DeviceArray((1, 16), np.uint16) for _ in range(2)]
    with pytest.raises(hy.HypError) as e:
        hy.qmatmul_group([a, b], x, 1, ys, stream)
    assert e.value.status_name == "INVALID_ARGUMENT"
    a.close()
    b.close()


def test_qmatmul_group_rmsnorm_rejects_a_misaligned_norm_weight(stream):
    """norm_weight is copied into LDS by 16-byte direct loads: a pointer off that alignment
    is refused on the host (INVALID_ARGUMENT) before any launch."""
    a = hy.QWeight.from_host(*syn.q4_weights(16, 128, seed=1243))
    x = dev(syn.activations(1, 128, seed=1244), stream)
    nw = dev(syn.bf16_bits(np.ones(136, np.float32)), stream)
    ys = [hy.DeviceArray((1, 16), np.uint16)]

    class Shifted:
        ptr = ctypes.c_void_p(nw.ptr.value + 2)

    with pytest.raises(hy.HypError) as e:
        hy.qmatmul_group([a], x, 1, ys, stream, rms_eps=1e-6, norm_weight=Shifted())
    assert e.value.status_name == "INVALID_ARGUMENT"
    for t in (a, x, nw, *ys):
        t.close()


# ---------------------------------------------------------------- prefill GEMM

@pytest.mark.parametrize("m", [512, 2048])
def test_gemm_prefill_projections_sampled(stream, m):
    """Prefill GEMM for the seven projections; output rows are checked on a sample of
    16 rows per projection (the fp64 oracle over all rows would take minutes)."""
    rng = np.random.default_rng(m)
    for i, (name, (n, k)) in enumerate(syn.LAYER_SHAPES.items()):
        say(f"gemm m={m} {name} n={n} k={k}")
        x = syn.activations(m, k, seed=400 + i)
        w, s, b = syn.q4_weights(n, k, seed=500 + i)
        y = run_qmatmul(w, s, b, x, stream)
        rows = np.sort(rng.choice(m, size=16, replace=False))
        rows[0], rows[-1] = 0, m - 1
        xs = x[rows]
        ref_bf16w = O.qmatmul_deq_f64(xs, w, s, b, mode=1)
        truth = O.qmatmul_f64(xs, w, s, b)
        assert syn.sig_rel(syn.bf16_to_f32(y[rows]), truth) <= 1e-2, name
        assert_within_bf16_rounding(y[rows], ref_bf16w, name)


@pytest.mark.parametrize("m", [512, 1024, 2048])
def test_gemm_grouped_qkv_layer_shapes(stream, m):
    """The grouped q/k/v call of a layer at prefill sizes ([4096|2048|2048, 3840] in one
    launch): m = 512 takes the 128 x 256 group-step kernel with 2 k splits, m = 1024 the
    same unsplit and m = 2048 the 256 x 256 one. Sampled rows against the fp64 product with
    the kernel's bf16 weights, and sig_rel <= 1e-2 against the fp64 truth."""
    k = 3840
    say(f"gemm grouped q/k/v m={m}")
    ws = [syn.q4_weights(n, k, seed=1600 + i) for i, n in enumerate((4096, 2048, 2048))]
    x = syn.activations(m, k, seed=1610 + m)
    ys = run_group(ws, x, stream)
    rng = np.random.default_rng(m + 7)
    rows = np.sort(rng.choice(m, size=10, replace=False))
    rows[0], rows[-1] = 0, m - 1
    for (w, s, b), y in zip(ws, ys):
        assert_within_bf16_rounding(y[rows], O.qmatmul_deq_f64(x[rows], w, s, b, mode=1), f"n={w.shape[0]}")
        assert syn.sig_rel(syn.bf16_to_f32(y[rows]), O.qmatmul_f64(x[rows], w, s, b)) <= 1e-2


def test_gemm_exact_integer_and_ragged_tiles(stream):
    rng = np.random.default_rng(8)
    for m, n, k in ((300, 200, 512), (257, 33, 64), (5, 1000, 3840), (2048, 40, 128)):
        say(f"gemm exact m={m} n={n} k={k}")
        x = rng.integers(-1, 2, size=(m, k)).astype(np.float32)
        codes = rng.integers(0, 16, size=(n, k)).astype(np.uint8)
        w = syn.pack_codes(codes)
        s = syn.bf16_bits(np.full((n, k // 64), 2.0**-7, np.float32))
        b = syn.bf16_bits(np.full((n, k // 64), -(2.0**-4), np.float32))
        exact = (x.astype(np.int64) @ (codes.astype(np.int64) - 8).T) * 2.0**-7
        y = run_qmatmul(w, s, b, syn.bf16_bits(x), stream)
        np.testing.assert_array_equal(y, syn.bf16_bits(exact.astype(np.float32)), err_msg=f"{m}x{n}x{k}")


def test_gemm_split_k_grouped_and_exact(stream):
    """Grids of at most one workgroup per CU split k (fp32 partials summed in order): a
    grouped call (n = 40, 24, 1000: the reduction maps workspace columns back to three
    outputs) with an odd group count (k = 4160), against the fp64 product with the
    kernel's bf16 weights; and exact integer inputs (300 x 200 x 4096, 4 splits of 8
    pairs), bit-exact."""
    m, k = 200, 4160
    ws = [syn.q4_weights(n, k, seed=1400 + n) for n in (40, 24, 1000)]
    x = syn.activations(m, k, seed=1410)
    say(f"split-k group m={m} k={k}")
    ys = run_group(ws, x, stream)
    for (w, s, b), y in zip(ws, ys):
        assert_within_bf16_rounding(y, O.qmatmul_deq_f64(x, w, s, b, mode=1), f"n={w.shape[0]}")
    rng = np.random.default_rng(14)
    m, n, k = 300, 200, 4096
    say(f"split-k exact m={m} n={n} k={k}")
    xi = rng.integers(-1, 2, size=(m, k)).astype(np.float32)
    codes = rng.integers(0, 16, size=(n, k)).astype(np.uint8)
    s2 = syn.bf16_bits(np.full((n, k // 64), 2.0**-7, np.float32))
    b2 = syn.bf16_bits(np.full((n, k // 64), -(2.0**-4), np.float32))
    exact = (xi.astype(np.int64) @ (codes.astype(np.int64) - 8).T) * 2.0**-7
    y2 = run_qmatmul(syn.pack_codes(codes), s2, b2, syn.bf16_bits(xi), stream)
    np.testing.assert_array_equal(y2, syn.bf16_bits(exact.astype(np.float32)))


@pytest.mark.parametrize("n,k", [(8200, 192), (8195, 320), (8200, 3840)])
def test_gemm_group_step_tiles(stream, n, k):
    """Grids of >= 0.9 workgroups per CU in 256 x 256 tiles select the 256-row group-step kernel: ragged m
    (2000 rows, the last row tile part-empty), n with a part-empty 16-row tile (8200) or
    n % 8 != 0 (8195: the element-wise store path), odd group counts (k = 192, 320).
    Sampled rows against the fp64 product with the kernel's bf16 weights, and all rows
    exact on integer inputs."""
    m = 2000
    say(f"gemm group-step m={m} n={n} k={k}")
    x = syn.activations(m, k, seed=1300 + k)
    w, s, b = syn.q4_weights(n, k, seed=1301 + n)
    y = run_qmatmul(w, s, b, x, stream)
    rng = np.random.default_rng(n + k)
    rows = np.sort(rng.choice(m, size=12, replace=False))
    rows[0], rows[-1] = 0, m - 1
    assert_within_bf16_rounding(y[rows], O.qmatmul_deq_f64(x[rows], w, s, b, mode=1), f"n={n} k={k}")
    # exact arithmetic over every row and column
    xi = rng.integers(-1, 2, size=(m, k)).astype(np.float32)
    codes = rng.integers(0, 16, size=(n, k)).astype(np.uint8)
    s2 = syn.bf16_bits(np.full((n, k // 64), 2.0**-7, np.float32))
    b2 = syn.bf16_bits(np.full((n, k // 64), -(2.0**-4), np.float32))
    exact = (xi.astype(np.int64) @ (codes.astype(np.int64) - 8).T) * 2.0**-7
    y2 = run_qmatmul(syn.pack_codes(codes), s2, b2, syn.bf16_bits(xi), stream)
    np.testing.assert_array_equal(y2, syn.bf16_bits(exact.astype(np.float32)), err_msg=f"exact n={n} k={k}")


@pytest.mark.parametrize("m,n,splits", [(1300, 6000, 1), (700, 2999, 4)])
def test_gemm_group_step_128_rows(stream, m, n, splits):
    """Mid-size grids select the 128 x 256 group-step kernel, unsplit (11 x 24 tiles) or
    with 4 k splits (6 x 12 tiles; n = 2999 is odd, so the split sums take the
    element-wise reduction): ragged m (the last 128-row tile part-empty), n not a multiple
    of 256, an odd group count (k = 4160: 65 groups, so the last pair is half empty).
    Sampled rows against the fp64 product with the kernel's bf16 weights, and exact
    integer inputs on sampled rows including the last row tile."""
    k = 4160
    say(f"gemm group-step 128 rows m={m} n={n} k={k} (splits {splits})")
    x = syn.activations(m, k, seed=1700 + m)
    w, s, b = syn.q4_weights(n, k, seed=1701 + n)
    y = run_qmatmul(w, s, b, x, stream)
    rng = np.random.default_rng(m + n)
    rows = np.sort(rng.choice(m, size=12, replace=False))
    rows[0], rows[-1] = 0, m - 1
    assert_within_bf16_rounding(y[rows], O.qmatmul_deq_f64(x[rows], w, s, b, mode=1), f"m={m} n={n}")
    xi = rng.integers(-1, 2, size=(m, k)).astype(np.float32)
    codes = rng.integers(0, 16, size=(n, k)).astype(np.uint8)
    s2 = syn.bf16_bits(np.full((n, k // 64), 2.0**-7, np.float32))
    b2 = syn.bf16_bits(np.full((n, k // 64), -(2.0**-4), np.float32))
    y2 = run_qmatmul(syn.pack_codes(codes), s2, b2, syn.bf16_bits(xi), stream)
    check = np.unique(np.concatenate([rows, np.arange(m - 20, m)]))
    exact = (xi[check].astype(np.float64) @ (codes.astype(np.float64) - 8).T) * 2.0**-7
    np.testing.assert_array_equal(y2[check], syn.bf16_bits(exact.astype(np.float32)), err_msg=f"exact m={m} n={n}")


@pytest.mark.parametrize("m,n,k", [(2048, 40, 128), (300, 200, 4096)])
def test_gemm_output_not_16_byte_aligned(stream, m, n, k):
    """y one element past a 16-byte boundary: the 16-byte store paths (the tile epilogue,
    and the 8-column split-k reduction for the 4-split 300 x 200 x 4096 call) fall back
    to element stores; results equal the aligned call's bit for bit."""
    import ctypes
    say(f"gemm unaligned y m={m} n={n} k={k}")
    x = syn.activations(m, k, seed=1800 + k)
    w, s, b = syn.q4_weights(n, k, seed=1801 + n)
    ref = run_qmatmul(w, s, b, x, stream)
    qw = hy.QWeight.from_host(w, s, b)
    xd = dev(x, stream)
    yd = hy.DeviceArray((m * n + 8,), np.uint16)
    yd.fill_zero(stream)
    hy.call("hyp_qmatmul", qw.handle, xd.ptr, m, ctypes.c_void_p(yd.ptr.value + 2), stream.handle)
    got = yd.to_host(stream)
    assert got[0] == 0 and np.all(got[1 + m * n:] == 0)
    np.testing.assert_array_equal(got[1:1 + m * n].reshape(m, n), ref)
    qw.close()


def test_gemm_group_step_split_k(stream):
    """A long k (129 groups) on a grid short of the CUs (8 x 12 tiles of 256 x 256) runs the
    256-row group-step kernel with k split 3 ways (22-pair ranges, the last covering 41
    groups and ending on a half pair): a grouped call over two segments (n = 1000, 2000) with ragged
    m = 2000, against the fp64 product with the kernel's bf16 weights on sampled rows; and
    exact integer inputs on one [3000, 8256] matrix, bit-exact on sampled rows including
    the part-empty last row tile."""
    m, k = 2000, 8256
    say(f"gemm group-step split-k m={m} k={k}")
    ws = [syn.q4_weights(n, k, seed=1500 + n) for n in (1000, 2000)]
    x = syn.activations(m, k, seed=1510)
    ys = run_group(ws, x, stream)
    rng = np.random.default_rng(k)
    rows = np.sort(rng.choice(m, size=12, replace=False))
    rows[0], rows[-1] = 0, m - 1
    for (w, s, b), y in zip(ws, ys):
        assert_within_bf16_rounding(y[rows], O.qmatmul_deq_f64(x[rows], w, s, b, mode=1), f"n={w.shape[0]}")
    n = 3000
    xi = rng.integers(-1, 2, size=(m, k)).astype(np.float32)
    codes = rng.integers(0, 16, size=(n, k)).astype(np.uint8)
    s2 = syn.bf16_bits(np.full((n, k // 64), 2.0**-7, np.float32))
    b2 = syn.bf16_bits(np.full((n, k // 64), -(2.0**-4), np.float32))
    y2 = run_qmatmul(syn.pack_codes(codes), s2, b2, syn.bf16_bits(xi), stream)
    check = np.unique(np.concatenate([rows, np.arange(m - 16, m)]))
    exact = (xi[check].astype(np.float64) @ (codes.astype(np.float64) - 8).T) * 2.0**-7   # integers < 2^17: exact
    np.testing.assert_array_equal(y2[check], syn.bf16_bits(exact.astype(np.float32)), err_msg="exact split-k group-step")


# ---------------------------------------------------------------- fused epilogues

def _assert_close_bits(got, ref, what, max_ulp=1):
    d = ulp_diff(got, ref)
    assert d.max() <= max_ulp, what
    assert np.count_nonzero(d) <= max(1, d.size // 1000), what


@pytest.mark.parametrize("m", [1, 4, 300])
def test_gate_up_gelu_fused(stream, m):
    """The fused gate/up against the oracle's bf16 GELU chain applied to gate and up
    launches, and against the chain applied to the fp64 truth.
    m <= 4: one decode launch, against separate gate and up launches. It may split a
    tile's k range differently, so its fp32 sums are the same terms in another order: a
    bf16 gate or up value can then round the other way (1 ulp), which the GELU chain and
    the product carry to at most 2 ulps, in at most 0.1% of the outputs here (deep in
    GELU's negative tail one gate ulp moves the output by many ulps).
    m > 4: the dual GEMM, against the grouped [gate, up] launch, which makes the same k
    split and sums: bit-exact."""
    n, k = 15360, 3840
    say(f"gate/up gelu m={m}")
    x = syn.activations(m, k, seed=600 + m)
    gw, gs, gb = syn.q4_weights(n, k, seed=601)
    uw, us, ub = syn.q4_weights(n, k, seed=602)
    gate = hy.QWeight.from_host(gw, gs, gb)
    up = hy.QWeight.from_host(uw, us, ub)
    xd = dev(x, stream)
    g = hy.DeviceArray((m, n), np.uint16)
    u = hy.DeviceArray((m, n), np.uint16)
    h = hy.DeviceArray((m, n), np.uint16)
    if m > 4:
        hy.qmatmul_group([gate, up], xd, m, [g, u], stream)
    else:
        hy.qmatmul(gate, xd, m, g, stream)
        hy.qmatmul(up, xd, m, u, stream)
    hy.qmlp_gate_up_gelu(gate, up, xd, m, h, stream)
    hb = h.to_host(stream)
    chain = O.gelu_tanh_mul(g.to_host(stream), u.to_host(stream))
    if m > 4:
        np.testing.assert_array_equal(hb, chain, err_msg=f"m={m}")
    else:
        _assert_close_bits(hb, chain, f"m={m}", max_ulp=2)
    rows = min(m, 8)
    g64 = O.qmatmul_f64(x[:rows], gw, gs, gb) if m <= 4 else O.qmatmul_deq_f64(x[:rows], gw, gs, gb, mode=1)
    u64 = O.qmatmul_f64(x[:rows], uw, us, ub) if m <= 4 else O.qmatmul_deq_f64(x[:rows], uw, us, ub, mode=1)
    truth = syn.bf16_to_f32(O.gelu_tanh_mul(syn.bf16_bits(g64.astype(np.float32)), syn.bf16_bits(u64.astype(np.float32))))
    rel = syn.sig_rel(syn.bf16_to_f32(hb[:rows]), truth)
    say(f"  gate/up gelu m={m}: sig_rel vs the chain on the fp64 gate and up = {rel:.2e} (bound 1e-2)")
    assert rel <= 1e-2


DUAL_CASES = [
    # n, k, m: the 256 x 256 group-step kernel; the 128 x 256 one; the pair-step kernel;
    # the pair-step kernel split 4 ways (the dual split-k reduce); an odd group count; a
    # ragged n; the smallest GEMM batch
    (15360, 3840, 2048),
    (15360, 3840, 512),
    (15360, 3840, 64),
    (512, 3840, 64),
    (384, 192, 40),
    (1000, 640, 33),
    (15360, 3840, 5),
]


@pytest.mark.parametrize("n,k,m", DUAL_CASES)
def test_gate_up_gelu_dual_gemm_equals_grouped_launch(stream, n, k, m):
    """At m > 4 hyp_qmlp_gate_up_gelu is one dual GEMM (gate and up tiles accumulated by
    the same wave, the gating in the epilogue). It picks the kernel and k split of the
    grouped [gate, up] GEMM and sums the same terms in the same order, so its output is
    the oracle's GELU chain over that launch's gate and up outputs, bit for bit."""
    say(f"dual gate/up gemm n={n} k={k} m={m}")
    x = syn.activations(m, k, seed=620 + m)
    gate = hy.QWeight.from_host(*syn.q4_weights(n, k, seed=621 + n))
    up = hy.QWeight.from_host(*syn.q4_weights(n, k, seed=622 + n))
    xd = dev(x, stream)
    g = hy.DeviceArray((m, n), np.uint16)
    u = hy.DeviceArray((m, n), np.uint16)
    h = hy.DeviceArray((m, n), np.uint16)
    hy.qmatmul_group([gate, up], xd, m, [g, u], stream)
    hy.qmlp_gate_up_gelu(gate, up, xd, m, h, stream)
    np.testing.assert_array_equal(h.to_host(stream), O.gelu_tanh_mul(g.to_host(stream), u.to_host(stream)))
    for a in (gate, up, xd, g, u, h):
        a.close()


@pytest.mark.parametrize("m", [1, 300])
def test_lm_head_softcap(stream, m):
    n, k = 32768, 3840
    say(f"lm head softcap m={m}")
    x = syn.activations(m, k, seed=700 + m)
    w, s, b = syn.q4_weights(n, k, seed=701)
    s = syn.bf16_bits(syn.bf16_to_f32(s) * np.float32(64.0))       # logits of magnitude ~30+
    b = syn.bf16_bits(syn.bf16_to_f32(b) * np.float32(64.0))
    plain = run_qmatmul(w, s, b, x, stream)
    capped = run_qmatmul(w, s, b, x, stream, softcap=30.0)
    assert np.max(np.abs(syn.bf16_to_f32(plain))) > 30.0
    # The head launch may split k differently from the plain launch (the same terms summed
    # in another order): a pre-cap logit can round the other way, at most 2 ulps after the cap.
    _assert_close_bits(capped, O.softcap(plain, 30.0), f"m={m}", max_ulp=2)


# ---------------------------------------------------------------- greedy sampling on the device

def _sample_rows(bits2d, stream, rows, vocab, row_offset=0):
    d = dev(bits2d, stream)
    out = hy.DeviceArray((max(rows, 1) * 3,), np.uint32)
    hy.sample_greedy(d, rows, vocab, out, stream, row_offset=row_offset)
    got = hy.greedy_samples(out, rows, stream)
    d.close()
    out.close()
    return got


def _assert_samples_equal(got, want, what):
    g_tok, g_val, g_tie = got
    w_tok, w_val, w_tie = want
    assert (g_tok, g_tie) == (w_tok, w_tie), f"{what}: {got} vs {want}"
    assert np.float32(g_val).tobytes() == np.float32(w_val).tobytes(), f"{what}: {got} vs {want}"


def _planted_logits(rng, rows, vocab):
    """Random bf16 logits with, per row, one of: a tie at the maximum (the later index
    must lose), NaN and +-inf entries, a near tie at gap 0.375 or 0.5, or nothing."""
    v = syn.bf16_bits((rng.standard_normal((rows, vocab)) * 6).astype(np.float32))
    for r in range(rows):
        kind = r % 4
        if vocab < 4:
            continue
        i, j = sorted(rng.choice(vocab, 2, replace=False))
        if kind == 1:
            v[r, i] = v[r, j] = syn.bf16_bits(np.float32([60.0]))[0]
        elif kind == 2:
            v[r, rng.integers(vocab)] = 0x7FC0
            v[r, rng.integers(vocab)] = 0xFF80
            v[r, i] = 0x7F80 if r % 8 == 2 else syn.bf16_bits(np.float32([70.0]))[0]
        elif kind == 3:
            v[r, j] = syn.bf16_bits(np.float32([64.0]))[0]
            v[r, i] = syn.bf16_bits(np.float32([63.625 if r % 8 == 3 else 63.5]))[0]
    return v


@pytest.mark.parametrize("vocab", [262144, 262143, 1000, 8, 7, 1])
def test_sample_greedy_matches_oracle(stream, vocab):
    """hyp_sample_greedy against the oracle's restatement of forward.cc:162-189, exactly
    (token, logit bits, near_tie), on 8 rows with planted ties, NaN, infinities and near
    ties; vocab % 8 != 0 takes the element-wise path; a row offset makes the start
    unaligned."""
    rng = np.random.default_rng(vocab)
    rows = 8
    say(f"sample_greedy vocab={vocab}")
    v = _planted_logits(rng, rows, vocab)
    got = _sample_rows(v, stream, rows, vocab)
    for r in range(rows):
        _assert_samples_equal(got[r], O.sample_greedy(v[r]), f"vocab={vocab} row={r}")
    got = _sample_rows(v, stream, rows - 1, vocab, row_offset=1)
    for r in range(rows - 1):
        _assert_samples_equal(got[r], O.sample_greedy(v[r + 1]), f"vocab={vocab} offset row={r + 1}")


def test_sample_greedy_many_rows(stream):
    """130 rows run as three passes over the stream's 64-row workspace; every row equals
    the oracle's scan."""
    rng = np.random.default_rng(130)
    rows, vocab = 130, 4104
    say(f"sample_greedy rows={rows} vocab={vocab}")
    v = _planted_logits(rng, rows, vocab)
    got = _sample_rows(v, stream, rows, vocab)
    for r in range(rows):
        _assert_samples_equal(got[r], O.sample_greedy(v[r]), f"row={r}")


def test_sample_greedy_degenerate_rows(stream):
    """All -inf, all NaN and vocab = 0 rows give token 0 with logit -inf and no near tie
    (the reference's initial values survive the scan); rows = 0 is a no-op."""
    say("sample_greedy degenerate rows")
    v = np.stack([np.full(4096, 0xFF80, np.uint16), np.full(4096, 0x7FC0, np.uint16)])
    for got in _sample_rows(v, stream, 2, 4096):
        _assert_samples_equal(got, (0, float("-inf"), False), "degenerate")
    for got in _sample_rows(np.zeros((2, 8), np.uint16), stream, 2, 0):
        _assert_samples_equal(got, (0, float("-inf"), False), "vocab=0")
    assert _sample_rows(v, stream, 0, 4096) == []


def test_lm_head_softcap_then_device_greedy(stream):
    """run_epilogue (model.cc:215-228) on the device: the tied head with softcap on m = 3
    rows of a [32768, 3840] table, then greedy sampling of the last row, equal to the
    oracle's sampler on that row of the kernel's own logits."""
    n, k, m = 32768, 3840, 3
    say("lm head softcap -> device greedy")
    x = syn.activations(m, k, seed=711)
    w, s, b = syn.q4_weights(n, k, seed=712)
    s = syn.bf16_bits(syn.bf16_to_f32(s) * np.float32(64.0))
    b = syn.bf16_bits(syn.bf16_to_f32(b) * np.float32(64.0))
    qw = hy.QWeight.from_host(w, s, b)
    xd = dev(x, stream)
    yd = hy.DeviceArray((m, n), np.uint16)
    hy.qmatmul(qw, xd, m, yd, stream, softcap=30.0)
    out = hy.DeviceArray((3,), np.uint32)
    hy.sample_greedy(yd, 1, n, out, stream, row_offset=m - 1)
    got = hy.greedy_samples(out, 1, stream)[0]
    logits = yd.to_host(stream)
    _assert_samples_equal(got, O.sample_greedy(logits[m - 1]), "head last row")
    assert got[1] <= 30.0
    for a in (qw, xd, yd, out):
        a.close()


# ---------------------------------------------------------------- residency (tiny artifact)

def test_qmodel_fixture_reference_weights_test(stream, fixture_dir):
    """weights_test.cc:101-139 on every projection of the reference's tiny artifact:
    x = 0.1 (M=4, and M=300 for the GEMM path) against dequantize+matmul at
    allclose(rtol=1e-3, atol=1e-2)."""
    model = hy.QModel(fixture_dir)
    tensors = st_reader.q4_tensors(fixture_dir)
    assert model.num_layers == 6
    with pytest.raises(hy.HypError) as err:
        model.linear(5, "v")
    assert err.value.status_name == "NOT_FOUND"
    for layer in range(6):
        for proj in ("q", "k", "v", "o", "gate", "up", "down"):
            if layer == 5 and proj == "v":
                continue
            sect = "mlp" if proj in ("gate", "up", "down") else "self_attn"
            w, s, b = tensors[f"language_model.model.layers.{layer}.{sect}.{proj}_proj"]
            qw = model.linear(layer, proj)
            n, k = qw.shape
            assert (n, k) == (w.shape[0], w.shape[1] * 8)
            ew, es, eb = qw.export()
            assert np.array_equal(ew, w) and np.array_equal(es, s) and np.array_equal(eb, b)
            for m in (4, 300):
                x = syn.bf16_bits(np.full((m, k), 0.1, np.float32))
                xd = dev(x, stream)
                yd = hy.DeviceArray((m, n), np.uint16)
                hy.qmatmul(qw, xd, m, yd, stream)
                ref = syn.bf16_to_f32(x) @ syn.bf16_to_f32(O.dequantize(w, s, b, mode=1)).T
                np.testing.assert_allclose(syn.bf16_to_f32(yd.to_host(stream)), ref, rtol=1e-3, atol=1e-2)
    emb = model.embed()
    ids = np.array([0, 5, 127, 64], np.uint32)
    out = hy.DeviceArray((ids.size, 128), np.uint16)
    hy.embed(emb, dev(ids, stream), ids.size, out, stream)
    w, s, b = tensors["language_model.model.embed_tokens"]
    ref = O.scale(O.dequantize(w, s, b, rows=ids), float(np.sqrt(np.float32(128))))
    np.testing.assert_array_equal(out.to_host(stream), ref)
    with pytest.raises(hy.HypError):
        hy.call("hyp_qweight_free", __import__("ctypes").byref(emb.handle))
    model.close()


def test_zero_rows_is_a_noop(stream):
    w, s, b = syn.q4_weights(64, 128, seed=9)
    qw = hy.QWeight.from_host(w, s, b)
    y = hy.DeviceArray((1, 64), np.uint16)
    y.fill_zero(stream)
    hy.qmatmul(qw, y, 0, y, stream)
    stream.synchronize()
    assert np.all(y.to_host(stream) == 0)


# ---------------------------------------------------------------- tiled layout edge cases

@pytest.mark.parametrize("k", [64, 192, 320])
def test_odd_group_counts_through_every_path(stream, k):
    """k/64 odd leaves the last pair of the tiled layout half empty: the skinny kernel
    (m <= 4), the GEMM (m > 4), export and embed must all ignore the missing group."""
    n = 40   # not a multiple of 16: the last row tile is partly empty too
    w, s, b = syn.q4_weights(n, k, seed=900 + k)
    qw = hy.QWeight.from_host(w, s, b)
    ew, es, eb = qw.export()
    assert np.array_equal(ew, w) and np.array_equal(es, s) and np.array_equal(eb, b)
    for m in (1, 3, 4, 5, 37):
        say(f"odd groups k={k} m={m}")
        x = syn.activations(m, k, seed=901 + m)
        xd = dev(x, stream)
        yd = hy.DeviceArray((m, n), np.uint16)
        hy.qmatmul(qw, xd, m, yd, stream)
        y = yd.to_host(stream)
        ref = O.qmatmul_deq_f64(x, w, s, b, mode=1) if m > 4 else O.qmatmul_f64(x, w, s, b)
        assert_within_bf16_rounding(y, ref, f"k={k} m={m}")
    ids = np.array([0, 39, 17, 16, 15], np.uint32)
    out = hy.DeviceArray((ids.size, k), np.uint16)
    hy.embed(qw, dev(ids, stream), ids.size, out, stream)
    ref = O.scale(O.dequantize(w, s, b, rows=ids), float(np.sqrt(np.float32(k))))
    np.testing.assert_array_equal(out.to_host(stream), ref)
    qw.close()


# ---------------------------------------------------------------- renormalisation

def test_rms_normalize_rows(stream):
    m, k = 5, 3840
    x = syn.activations(m, k, seed=950)
    x[2] = syn.bf16_bits(syn.bf16_to_f32(x[2]) * np.float32(1e3))   # very different row scales
    x[3] = syn.bf16_bits(syn.bf16_to_f32(x[3]) * np.float32(1e-3))
    xd = dev(x, stream)
    yd = hy.DeviceArray((m, k), np.uint16)
    hy.rms_normalize(xd, m, k, yd, stream, eps=1e-6)
    got = syn.bf16_to_f32(yd.to_host(stream)).astype(np.float64)
    xf = syn.bf16_to_f32(x).astype(np.float64)
    ref = xf / np.sqrt(np.mean(xf * xf, axis=1, keepdims=True) + 1e-6)
    # one bf16 rounding of the product plus fp32 statistics
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-8 * 1.01 + 1e-30)
    hy.rms_normalize(xd, m, k, xd, stream, eps=1e-6)   # in place
    np.testing.assert_array_equal(xd.to_host(stream), yd.to_host(stream))


@pytest.mark.parametrize("k", [1000, 19200])
def test_rms_normalize_other_widths(stream, k):
    """k not a multiple of 64 (the element-wise kernel) and more 64-wide units per row
    than threads (19200 = 300 units: units loaded twice)."""
    m = 3
    x = syn.activations(m, k, seed=960 + k)
    yd = hy.DeviceArray((m, k), np.uint16)
    hy.rms_normalize(dev(x, stream), m, k, yd, stream, eps=1e-5)
    got = syn.bf16_to_f32(yd.to_host(stream)).astype(np.float64)
    xf = syn.bf16_to_f32(x).astype(np.float64)
    ref = xf / np.sqrt(np.mean(xf * xf, axis=1, keepdims=True) + 1e-5)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0**-8 * 1.01 + 1e-30)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5])
def test_qmatmul_group_rmsnorm_equals_two_calls(stream, m):
    """hyp_qmatmul_group_rmsnorm == hyp_rms_normalize then hyp_qmatmul_group, bit for bit
    (one launch with the normalisation in LDS at m <= 4, a temporary above), x unchanged,
    and within the qmatmul bars of the fp64 product of the normalised rows."""
    k = 3840
    ws = [syn.q4_weights(n, k, seed=1250 + i) for i, n in enumerate((4096, 2048, 2048))]
    qws = [hy.QWeight.from_host(*w) for w in ws]
    x = syn.activations(m, k, seed=1260 + m)
    x[0] = syn.bf16_bits(syn.bf16_to_f32(x[0]) * np.float32(37.0))   # rows of different scale
    xd = dev(x, stream)
    fused = [hy.DeviceArray((m, w[0].shape[0]), np.uint16) for w in ws]
    hy.qmatmul_group(qws, xd, m, fused, stream, rms_eps=1e-6)
    np.testing.assert_array_equal(xd.to_host(stream), x)
    xn = hy.DeviceArray((m, k), np.uint16)
    hy.rms_normalize(xd, m, k, xn, stream, eps=1e-6)
    sep = [hy.DeviceArray((m, w[0].shape[0]), np.uint16) for w in ws]
    hy.qmatmul_group(qws, xn, m, sep, stream)
    xn_host = xn.to_host(stream)
    for (w, s, b), f, g, name in zip(ws, fused, sep, ("q", "k", "v")):
        say(f"group rmsnorm m={m} {name}")
        yf = f.to_host(stream)
        np.testing.assert_array_equal(yf, g.to_host(stream), err_msg=name)
        truth = O.qmatmul_f64(xn_host, w, s, b) if m <= 4 else O.qmatmul_deq_f64(xn_host, w, s, b, mode=1)
        assert_within_bf16_rounding(yf, truth, name)
    for q in qws:
        q.close()


@pytest.mark.parametrize("m,k,ns", [(4, 10240, (512, 256, 256)), (1, 10240, (512, 256, 256)),
                                    (4, 8192, (256, 64, 64)), (3, 3840, (128, 64, 64)),
                                    (1, 3840, (8192, 512)), (4, 3840, (8192, 512)),
                                    (2, 1024, (256, 64, 64)), (4, 1024, (1024, 256)), (3, 1280, (512,))])
@pytest.mark.parametrize("weighted", [False, True])
def test_qmatmul_group_rmsnorm_launch_shapes(stream, m, k, ns, weighted):
    """The normalising q/k/v launch in the workgroup shapes its launcher picks for other
    widths and grids - more (row, group) units than an 8-wave workgroup has threads (m = 4,
    k = 10240: 640 units), exactly as many (k = 8192), a grid of a few tiles, more waves
    than one round of 8-wave workgroups holds (the 12B's global q/k: 544 tiles at 4 splits,
    16-wave workgroups scaling x chunk by chunk), and the prologue with each unit spread over
    four lanes at several rows (m x k / 64 <= 64 units: 32, 64 and 60), with and without
    the norm's learned weight - equals hyp_rms_normalize then hyp_qmatmul_group, bit for bit."""
    ws = [syn.q4_weights(n, k, seed=1270 + i) for i, n in enumerate(ns)]
    qws = [hy.QWeight.from_host(*w) for w in ws]
    x = syn.activations(m, k, seed=1280 + m)
    xd = dev(x, stream)
    say(f"group rmsnorm m={m} k={k} n={ns} weighted={weighted}")
    nw = dev(syn.bf16_bits(1.0 + 0.2 * np.random.default_rng(k).standard_normal(k).astype(np.float32)), stream) \
        if weighted else None
    fused = [hy.DeviceArray((m, w[0].shape[0]), np.uint16) for w in ws]
    hy.qmatmul_group(qws, xd, m, fused, stream, rms_eps=1e-6, norm_weight=nw)
    xn = hy.DeviceArray((m, k), np.uint16)
    hy.rms_normalize(xd, m, k, xn, stream, eps=1e-6, weight=nw)
    sep = [hy.DeviceArray((m, w[0].shape[0]), np.uint16) for w in ws]
    hy.qmatmul_group(qws, xn, m, sep, stream)
    xn_host = xn.to_host(stream)
    for (w, s, b), f, g, name in zip(ws, fused, sep, ("q", "k", "v")):
        yf = f.to_host(stream)
        np.testing.assert_array_equal(yf, g.to_host(stream), err_msg=name)
        assert_within_bf16_rounding(yf, O.qmatmul_f64(xn_host, w, s, b), name)
    for a in qws + fused + sep + [xd, xn] + ([nw] if weighted else []):
        a.close()


# ---------------------------------------------------------------- graph capture

def test_graph_capture_replays_match_eager(stream):
    """A captured decode-style chain (GEMV, fused gate/up, GEMV, renormalise, softcap LM
    head) replayed several times, with eager work and synchronisation between the
    replays; every replay's outputs equal the eager run's."""
    k = 256
    shapes = {"a": (512, k), "gate": (384, k), "up": (384, k), "down": (k, 384), "head": (1000, k)}
    ws = {name: syn.q4_weights(n, kk, seed=960 + i) for i, (name, (n, kk)) in enumerate(shapes.items())}
    qws = {name: hy.QWeight.from_host(*v) for name, v in ws.items()}
    m = 2
    x0 = syn.activations(m, k, seed=970)
    h = dev(x0, stream)
    a = hy.DeviceArray((m, 512), np.uint16)
    g = hy.DeviceArray((m, 384), np.uint16)
    logits = hy.DeviceArray((m, 1000), np.uint16)

    def chain():
        hy.qmatmul(qws["a"], h, m, a, stream)
        hy.qmlp_gate_up_gelu(qws["gate"], qws["up"], h, m, g, stream)
        hy.qmatmul(qws["down"], g, m, h, stream)
        hy.rms_normalize(h, m, k, h, stream)
        hy.qmatmul(qws["head"], h, m, logits, stream, softcap=30.0)

    chain()
    eager = (a.to_host(stream), g.to_host(stream), h.to_host(stream), logits.to_host(stream))
    h.upload(x0, stream)
    with hy.Graph.capture(stream) as graph:
        chain()
    for rep in range(4):
        h.upload(x0, stream)                       # eager work between replays
        scratch = hy.DeviceArray((m, 512), np.uint16)
        hy.qmatmul(qws["a"], h, m, scratch, stream)
        stream.synchronize()
        graph.launch(stream)
        stream.synchronize()
        got = (a.to_host(stream), g.to_host(stream), h.to_host(stream), logits.to_host(stream))
        for e, gt, name in zip(eager, got, ("a", "gate/up", "h", "logits")):
            np.testing.assert_array_equal(gt, e, err_msg=f"replay {rep}: {name}")
        scratch.close()
    graph.close()
    for q in qws.values():
        q.close()
