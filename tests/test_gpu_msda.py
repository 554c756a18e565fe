"""MSDA forward on the GPU vs the float64 CPU oracle (oracle/msda.py), through the
reference-shaped API (msda_opt2.ms_deform_attn_forward -> _modulated_deform_conv_ext
.forward -> libbevk.so bevk_msda_forward).

Full-size BASELINE configurations run whole on the GPU and are checked on a random
subset of queries (each query's output depends only on its own locations/weights), plus
size-independent properties over the whole output (linearity in value and in attn)."""
import pytest
import torch

from _tol import check
from oracle import inputs
from oracle import msda as om

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _api():
    import msda_opt2
    return msda_opt2


def _run(d, dtype, **kw):
    dev = torch.device("cuda")
    out = _api().ms_deform_attn_forward(
        d["value"].to(dtype).to(dev), d["spatial_shapes"].to(dev),
        d["level_start_index"].to(dev), d["sampling_loc"].to(dtype).to(dev),
        d["attn_weight"].to(dtype).to(dev), **kw)
    torch.cuda.synchronize()
    return out.cpu()


def _ref(d, dtype, q_idx=None):
    """Oracle on the dtype-rounded inputs, in float64; optionally on a query subset."""
    v = d["value"].to(dtype).double()
    loc = d["sampling_loc"].to(dtype).double()
    att = d["attn_weight"].to(dtype).double()
    if q_idx is not None:
        loc = loc[:, q_idx]
        att = att[:, q_idx]
    return om.forward(v, d["spatial_shapes"], d["level_start_index"], loc, att)


@pytest.mark.parametrize("dtype", DTYPES, ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("cfg", ["msda_detr", "msda_tsa", "msda_sca"])
def test_configs_reduced(cfg, dtype):
    d = inputs.msda_inputs(cfg, scale_q=0.02)
    out = _run(d, dtype)
    assert out.dtype == dtype
    check(out, _ref(d, dtype), dtype, f"{cfg} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES, ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("cfg", ["msda_detr", "msda_tsa", "msda_sca"])
def test_configs_full_size(cfg, dtype):
    d = inputs.msda_inputs(cfg)
    out = _run(d, dtype)
    nq = d["sampling_loc"].shape[1]
    g = torch.Generator().manual_seed(123)
    q_idx = torch.randperm(nq, generator=g)[:400].sort().values
    q_idx = torch.cat([q_idx, torch.tensor([0, nq - 1])]).unique()
    check(out[:, q_idx], _ref(d, dtype, q_idx), dtype, f"{cfg} full {dtype}")


@pytest.mark.parametrize("dtype", DTYPES, ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("geom", [
    # batch, heads, num_query, shapes, points: large enough for the LDS-cached kernel
    # (16-bit types; fp32 runs the per-sample kernel with slice streaming)
    (3, 2, 11001, [(64, 90), (32, 45), (16, 23), (8, 12)], 8),   # level 1 partly cached,
    #   6 slices -> each slice split into query ranges over the 8 XCDs
    (1, 8, 8193, [(40, 70), (20, 35), (10, 18), (5, 9)], 4),      # 8 slices, DETR points
])
def test_cached_kernel_whole_output(geom, dtype):
    """Every query against the one-thread-per-element kernel (an independent code path),
    a subset against the float64 oracle; 40% of the samples lie outside the image."""
    b, nh, nq, shapes, npnt = geom
    d = inputs.msda_random(b, shapes, nq, nh, 32, npnt, seed=11, loc_lo=-0.25, loc_hi=1.25)
    # Exact pixel centres, edges and gates on a few queries.
    loc = d["sampling_loc"]
    loc[0, 0] = 0.0
    loc[0, 1] = 1.0
    H0, W0 = shapes[0]
    loc[0, 2, :, :, :, 0] = (W0 - 0.5) / W0
    loc[0, 2, :, :, :, 1] = 0.5 / H0
    out = _run(d, dtype)
    gen = _run(d, dtype, force_generic=True)
    if dtype == torch.float32:
        torch.testing.assert_close(out, gen, rtol=1e-5, atol=1e-5)
    else:
        check(out.double(), gen.double(), dtype, f"cached vs generic {geom}")
    g = torch.Generator().manual_seed(5)
    q_idx = torch.randperm(nq, generator=g)[:300].sort().values
    q_idx = torch.cat([q_idx, torch.tensor([0, 1, 2, nq - 1])]).unique()
    check(out[:, q_idx], _ref(d, dtype, q_idx), dtype, f"cached {geom}")


@pytest.mark.parametrize("dtype", DTYPES, ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("geom", [
    # batch, heads, num_query, shapes, points: below the LDS-cached kernel's size, so the
    # per-sample kernel runs every dtype, with 1024-2048 workgroups per slice: its first 64
    # workgroups per slice stream the slice's value lines and records (two heads per slice
    # in 16-bit types); query counts off the 64-way split, a short slice (S < 64 * 8)
    (1, 8, 4097, [(40, 52), (20, 26), (10, 13), (5, 7)], 8),
    (2, 4, 2111, [(12, 20), (6, 10), (3, 5), (2, 3)], 4),
])
def test_streaming_slices_whole_output(geom, dtype):
    """Every query against the one-thread-per-element kernel, a subset against the oracle,
    on launches where the per-sample kernel streams each slice into the cache first."""
    b, nh, nq, shapes, npnt = geom
    d = inputs.msda_random(b, shapes, nq, nh, 32, npnt, seed=41, loc_lo=-0.2, loc_hi=1.2)
    out = _run(d, dtype)
    gen = _run(d, dtype, force_generic=True)
    if dtype == torch.float32:
        torch.testing.assert_close(out, gen, rtol=1e-5, atol=1e-5)
    else:
        check(out.double(), gen.double(), dtype, f"streaming vs generic {geom}")
    g = torch.Generator().manual_seed(6)
    q_idx = torch.randperm(nq, generator=g)[:200].sort().values
    q_idx = torch.cat([q_idx, torch.tensor([0, nq - 1])]).unique()
    check(out[:, q_idx], _ref(d, dtype, q_idx), dtype, f"streaming {geom}")


def _tsa_like(b, H, W, sigma, seed, heads=8, points=4, extra=0):
    """Queries = the cells of one H x W grid (row-major), locations = cell centre + N(0, sigma)
    in normalised units, as BEVFormer temporal self-attention. extra > 0 appends unused value
    positions (spatial_size != H * W), which the tiled kernel must take in index order."""
    g = torch.Generator().manual_seed(seed)
    S = H * W + extra
    nq = S
    value = torch.randn(b, S, heads, 32, generator=g)
    q = torch.arange(nq)
    ref = torch.stack([((q % W).double() + 0.5) / W, ((q // W).double() + 0.5) / H], -1).float()
    loc = ref.view(1, nq, 1, 1, 1, 2).expand(b, nq, heads, 1, points, 2).clone()
    loc += sigma * torch.randn(b, nq, heads, 1, points, 2, generator=g)
    attn = torch.softmax(torch.randn(b, nq, heads, points, generator=g), -1)
    return dict(value=value, spatial_shapes=torch.tensor([[H, W]], dtype=torch.int64),
                level_start_index=torch.tensor([0], dtype=torch.int64),
                sampling_loc=loc.contiguous(), attn_weight=attn.view(b, nq, heads, 1, points))


@pytest.mark.parametrize("dtype", DTYPES, ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("geom", [
    # batch, H, W, sigma, extra positions
    (2, 40, 37, 0.01, 0),    # partial tiles on both edges, samples near their cell
    (1, 33, 50, 0.15, 0),    # wide offsets: many corners outside the staged neighbourhood
    (2, 16, 16, 0.01, 0),    # a single tile
    (1, 10, 12, 0.05, 10),   # spatial_size != H * W: queries taken in index order
])
def test_tsa_tiled(geom, dtype):
    """Single-level self-attention over a grid (the tiled kernel): every query against the
    float64 oracle and, in fp32, against the one-thread-per-element kernel."""
    b, H, W, sigma, extra = geom
    d = _tsa_like(b, H, W, sigma, seed=21, extra=extra)
    # Exact cell centres, image corners and far-outside samples on a few queries.
    loc = d["sampling_loc"]
    loc[0, 0] = 0.0
    loc[0, 1] = 1.0
    loc[0, 2, :, :, :, 0] = 5.0
    out = _run(d, dtype)
    check(out, _ref(d, dtype), dtype, f"tsa tiled {geom}")
    if dtype == torch.float32:
        gen = _run(d, dtype, force_generic=True)
        torch.testing.assert_close(out, gen, rtol=1e-5, atol=1e-5)


def test_sca_full_linearity():
    """Whole-output properties at the full SCA size: out is linear in value and in attn."""
    d = inputs.msda_inputs("msda_sca")
    base = _run(d, torch.float32)
    d2 = dict(d, value=d["value"] * 2.0)
    torch.testing.assert_close(_run(d2, torch.float32), base * 2.0, rtol=1e-6, atol=1e-6)
    d3 = dict(d, attn_weight=d["attn_weight"] * 0.5)
    torch.testing.assert_close(_run(d3, torch.float32), base * 0.5, rtol=1e-6, atol=1e-6)
    assert torch.isfinite(base).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.float64],
                         ids=["fp32", "fp16", "fp64"])
def test_force_generic(dtype):
    d = inputs.msda_inputs("msda_sca", scale_q=0.01, batch=2)
    out = _run(d, dtype, force_generic=True)
    check(out, _ref(d, dtype), dtype, "generic")


@pytest.mark.parametrize("geom", [
    # batch, shapes, num_query, heads, head_dim, points
    (2, [(7, 9), (4, 5), (2, 3)], 33, 4, 32, 5),      # D=32, runtime L/P
    (1, [(11, 13)], 17, 8, 16, 3),                     # D=16
    (3, [(6, 7), (3, 4)], 25, 2, 64, 2),               # D=64
    (2, [(5, 5), (9, 4)], 9, 3, 128, 4),               # D=128, odd heads
    (2, [(8, 6)], 13, 5, 24, 3),                       # D=24 -> generic kernel
    (1, [(1, 1), (2, 1)], 5, 8, 32, 8),                # 1-pixel levels
])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_geometries(geom, dtype):
    b, shapes, nq, nh, hd, npnt = geom
    d = inputs.msda_random(b, shapes, nq, nh, hd, npnt, seed=7, loc_lo=-0.3, loc_hi=1.3)
    out = _run(d, dtype)
    check(out, _ref(d, dtype), dtype, f"geom {geom}")


def test_edge_locations():
    """Pixel centres return the pixel, loc 0/1 give half-weight edges, far-out samples
    are zero, loc exactly at the -1 / H gates."""
    shapes = [(4, 6), (3, 5)]
    b, nq, nh, hd, npnt = 1, 8, 8, 32, 4
    d = inputs.msda_random(b, shapes, nq, nh, hd, npnt, seed=3)
    loc = d["sampling_loc"]
    loc[0, 0, :, 0, 0] = torch.tensor([(2 + 0.5) / 6, (1 + 0.5) / 4])   # pixel centre
    loc[0, 1, :, :, :] = 0.0                                           # corner (x=0, y=0)
    loc[0, 2, :, :, :] = 1.0                                           # corner (x=1, y=1)
    loc[0, 3, :, :, :] = 5.0                                           # far outside
    loc[0, 4, :, :, :] = -5.0
    loc[0, 5, :, 0, :, 1] = -0.5 / 4                                   # h_im exactly -1
    loc[0, 6, :, 0, :, 0] = (6 + 0.5) / 6                              # w_im exactly W
    out = _run(d, torch.float32)
    check(out, _ref(d, torch.float32), torch.float32, "edges")
    assert torch.all(out[0, 3] == 0) and torch.all(out[0, 4] == 0)


def test_empty_and_single():
    d = inputs.msda_random(2, [(3, 3)], 1, 8, 32, 4, seed=5)
    check(_run(d, torch.float32), _ref(d, torch.float32), torch.float32, "Lq=1")
    d0 = inputs.msda_random(2, [(3, 3)], 1, 8, 32, 4, seed=5)
    d0["sampling_loc"] = d0["sampling_loc"][:, :0].contiguous()
    d0["attn_weight"] = d0["attn_weight"][:, :0].contiguous()
    out = _run(d0, torch.float32)
    assert out.shape == (2, 0, 256)


def test_im2col_step_contract():
    d = inputs.msda_random(6, [(5, 7), (3, 4)], 11, 8, 32, 4, seed=9)
    ref = _ref(d, torch.float32)
    for step in (1, 2, 3, 6, 64):
        check(_run(d, torch.float32, im2col_step=step), ref, torch.float32, f"step {step}")
    with pytest.raises(RuntimeError, match="batch must divide im2col_step"):
        _run(d, torch.float32, im2col_step=4)


def test_on_side_stream():
    """The kernel is enqueued on torch's current stream."""
    d = inputs.msda_inputs("msda_tsa", scale_q=0.01)
    dev = torch.device("cuda")
    args = [d["value"].to(dev), d["spatial_shapes"].to(dev), d["level_start_index"].to(dev),
            d["sampling_loc"].to(dev), d["attn_weight"].to(dev)]
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        out = _api().ms_deform_attn_forward(*args)
    s.synchronize()
    check(out.cpu(), _ref(d, torch.float32), torch.float32, "side stream")


def test_non_contiguous_rejected():
    d = inputs.msda_random(2, [(3, 3)], 4, 8, 32, 4, seed=5)
    dev = torch.device("cuda")
    v = d["value"].to(dev).transpose(1, 2)
    with pytest.raises(RuntimeError, match="value must be contiguous"):
        _api().ms_deform_attn_forward(v, d["spatial_shapes"].to(dev),
                                      d["level_start_index"].to(dev),
                                      d["sampling_loc"].to(dev), d["attn_weight"].to(dev))


def _exact_centre(n):
    """Index i < n - 1 whose pixel centre (i + 0.5) / n is a dyadic fraction with at most
    8 significant bits (exact in fp32, fp16 and bf16), so the sample lands on the centre."""
    from fractions import Fraction
    for i in range(n - 1):
        fr = Fraction(2 * i + 1, 2 * n)
        if fr.denominator & (fr.denominator - 1) == 0 and fr.numerator < 256:
            return i, float(fr)
    raise ValueError(f"no exact pixel centre for size {n}")


def _poison(d, seed):
    """NaN / +Inf in value, following the reference's read rule (ms_deform_attn_kernels.cuh
    :7-49): a corner inside the level is read whatever its bilinear weight (0 * NaN = NaN,
    0 * Inf = NaN), a corner outside it contributes exactly 0 and is never read.
      * query 0, head 0 samples the exact centre of a level-0 pixel (y, x) at every point
        (its other levels far outside); value is finite at the sample's weighted corner and
        NaN at pixel (y + 1, x + 1), an in-bounds corner of weight 0 -> NaN;
      * query 1, head 1 samples far outside every level; value is NaN at level-0 pixel
        (0, 0) of head 1, where a clamped read would land -> output exactly 0;
      * a few random (position, head) rows of every level hold NaN or +Inf."""
    g = torch.Generator().manual_seed(seed)
    v, loc = d["value"], d["sampling_loc"]
    B, S, NH, D = v.shape
    shapes = d["spatial_shapes"].tolist()
    starts = d["level_start_index"].tolist()
    H0, W0 = shapes[0]
    for l, ((H, W), start) in enumerate(zip(shapes, starts)):
        for b in range(B):
            pos = start + torch.randint(0, H * W, (4,), generator=g)
            heads = torch.randint(0, NH, (4,), generator=g)
            for k in range(4):
                v[b, pos[k], heads[k], :] = float("nan") if k < 2 else float("inf")
    y, ly = _exact_centre(H0)
    x, lx = _exact_centre(W0)
    for p in (y * W0 + x, y * W0 + x + 1, (y + 1) * W0 + x):   # the sample's other corners
        v[0, p, 0, :] = 1.0
    v[0, (y + 1) * W0 + x + 1, 0, :] = float("nan")
    loc[0, 0, 0] = -5.0                                          # other levels: outside
    loc[0, 0, 0, 0, :, 0] = lx
    loc[0, 0, 0, 0, :, 1] = ly
    v[0, 0, 1, :] = float("nan")
    loc[0, 1, 1] = -5.0
    return d


@pytest.mark.parametrize("dtype", DTYPES, ids=["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("kind", ["wave", "generic", "cached", "cached_fixed", "tsa_tiled"])
def test_nonfinite_value(kind, dtype):
    """NaN and Inf in value give NaN / Inf exactly where the float64 oracle does, and the
    finite outputs match it to tolerance. 'cached' has three levels in LDS (run-time
    layout in 16-bit types, the per-sample kernel in fp32), 'cached_fixed' the two
    coarsest (the fixed-layout body in 16-bit types)."""
    force_generic = kind == "generic"
    if kind in ("wave", "generic"):
        d = inputs.msda_random(2, [(6, 8), (3, 5), (2, 3), (2, 2)], 50, 8, 32, 4, seed=31,
                               loc_lo=-0.3, loc_hi=1.3)
    elif kind == "cached":
        d = inputs.msda_random(3, [(64, 90), (32, 45), (16, 23), (8, 12)], 11001, 2, 32, 8,
                               seed=32, loc_lo=-0.25, loc_hi=1.25)
    elif kind == "cached_fixed":
        d = inputs.msda_random(1, [(116, 200), (58, 100), (29, 50), (15, 25)], 8192, 8, 32, 8,
                               seed=33, loc_lo=-0.2, loc_hi=1.2)
    else:
        d = _tsa_like(2, 40, 37, 0.01, seed=34)
    _poison(d, seed=35)
    nq = d["sampling_loc"].shape[1]
    out = _run(d, dtype, force_generic=force_generic).double()
    if nq > 4000:
        g = torch.Generator().manual_seed(36)
        q_idx = torch.cat([torch.randperm(nq, generator=g)[:300],
                           torch.tensor([0, 1, nq - 1])]).unique()
        out = out[:, q_idx]
        ref = _ref(d, dtype, q_idx)
    else:
        ref = _ref(d, dtype)
    what = f"nonfinite {kind} {dtype}"
    assert torch.equal(torch.isnan(out), torch.isnan(ref)), f"{what}: NaN pattern"
    assert torch.equal(torch.isinf(out), torch.isinf(ref)), f"{what}: Inf pattern"
    assert torch.equal(out[torch.isinf(ref)], ref[torch.isinf(ref)]), f"{what}: Inf sign"
    fin = torch.isfinite(ref)
    check(out[fin], ref[fin], dtype, what)
    D = 32
    assert torch.isnan(out[0, 0, :D]).all(), f"{what}: zero-weight NaN corner not read"
    assert (out[0, 1, D:2 * D] == 0).all(), f"{what}: out-of-range sample not exactly 0"
    assert 0.05 < fin.double().mean().item() < 0.999, f"{what}: degenerate poison pattern"
