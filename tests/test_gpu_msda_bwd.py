"""MSDA backward on the GPU vs the float64 CPU oracle (oracle/msda.py backward, pinned
against autograd and finite differences), through the reference-shaped API
(msda_opt2.ms_deform_attn_backward -> _modulated_deform_conv_ext.backward -> libbevk.so
bevk_msda_backward).

Reduced BASELINE configurations are compared whole. At full size, grad_sampling_loc and
grad_attn_weight of a random query subset are compared with the oracle run on that
subset (they depend only on the query's own data), and the whole of grad_value and
grad_attn_weight through the identities of a function linear in value and in attn:
  sum(grad_value * value) = sum(grad_output * out) = sum(grad_attn * attn)."""
import pytest
import torch

from _tol import check
from oracle import inputs
from oracle import msda as om

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
IDS = ["fp32", "fp16", "bf16"]
DEV = torch.device("cuda")


def _api():
    import msda_opt2
    return msda_opt2


def _grad_output(d, seed=11, dtype=torch.float32):
    B, Lq, NH = d["sampling_loc"].shape[:3]
    D = d["value"].shape[-1]
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, Lq, NH * D, generator=g).to(dtype)


def _dev(d, dtype):
    return dict(value=d["value"].to(dtype).to(DEV), spatial_shapes=d["spatial_shapes"].to(DEV),
                level_start_index=d["level_start_index"].to(DEV),
                sampling_loc=d["sampling_loc"].to(dtype).to(DEV),
                attn_weight=d["attn_weight"].to(dtype).to(DEV))


def _run(d, go, dtype, **kw):
    dd = _dev(d, dtype)
    gv, gl, ga = _api().ms_deform_attn_backward(**dd, grad_output=go.to(dtype).to(DEV), **kw)
    torch.cuda.synchronize()
    return gv.cpu(), gl.cpu(), ga.cpu()


def _ref(d, go, dtype, q_idx=None):
    """Oracle backward in float64 on the dtype-rounded inputs, at the sampling coordinates
    the fp32 algorithm defines (h_im = loc*H - 0.5 rounded to fp32, as the reference's
    `float h_im` and the kernel's fused multiply-add compute it: grad_sampling_loc scales
    the coordinate's rounding error by W, above the 1e-4 bound); optionally a query subset
    (its grad_value then covers only that subset's samples)."""
    v = d["value"].to(dtype).double()
    loc = d["sampling_loc"].to(dtype).double()
    att = d["attn_weight"].to(dtype).double()
    g = go.to(dtype).double()
    if q_idx is not None:
        loc, att, g = loc[:, q_idx], att[:, q_idx], g[:, q_idx]
    coord = None if dtype == torch.float64 else torch.float32
    return om.backward(v, d["spatial_shapes"], d["level_start_index"], loc, att, g,
                       coord_dtype=coord)


def _check3(got, ref, dtype, what):
    for name, x, r in zip(("grad_value", "grad_sampling_loc", "grad_attn_weight"), got, ref):
        assert x.dtype == dtype, f"{what} {name}: dtype {x.dtype}"
        check(x, r, dtype, f"{what} {name}")


def _run_workspace(d, go, dtype, ws_bytes, gv_init=0.0):
    """bevk_msda_backward through the C ABI with a workspace of ws_bytes: below
    bevk_msda_backward_workspace_bytes (the sorted path's buffers), D = 32 takes the owner
    kernels for grid queries and the atomic kernels (msda_col2im_d32_kernel +
    msda_coarse_gv_kernel) otherwise; fp32 needs no workspace, 16-bit types the fp32
    grad_value accumulator. grad_value starts at gv_init (fp32 adds to it)."""
    import _bevk as b
    dd = _dev(d, dtype)
    value, loc = dd["value"], dd["sampling_loc"]
    B, S, NH, D = value.shape
    Lq, L, P = loc.shape[1], loc.shape[3], loc.shape[4]
    g4 = go.to(dtype).to(DEV).view(B, Lq, NH, D)
    gv = torch.full_like(value, gv_init)
    gl = torch.empty_like(loc)
    ga = torch.empty_like(dd["attn_weight"])
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    b.call("bevk_msda_backward", b.dtype_code(value), b.ptr(value), b.ptr(dd["spatial_shapes"]),
           b.ptr(dd["level_start_index"]), b.ptr(loc), b.ptr(dd["attn_weight"]), b.ptr(g4),
           *g4.stride(), B, S, NH, D, L, Lq, P, 64, 0, b.ptr(gv), b.ptr(gl), b.ptr(ga),
           b.ptr(ws), ws_bytes, b.stream_of(value))
    torch.cuda.synchronize()
    return gv.cpu(), gl.cpu(), ga.cpu()


def _accumulator_bytes(d, dtype):
    return 0 if dtype == torch.float32 else d["value"].numel() * 4


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("cfg", ["msda_detr", "msda_tsa", "msda_sca"])
def test_configs_reduced(cfg, dtype):
    d = inputs.msda_inputs(cfg, scale_q=0.02)
    go = _grad_output(d)
    _check3(_run(d, go, dtype), _ref(d, go, dtype), dtype, f"{cfg} {dtype}")


def test_fp64():
    d = inputs.msda_inputs("msda_sca", scale_q=0.01, batch=2)
    go = _grad_output(d)
    got = _run(d, go, torch.float64)
    for x, r in zip(got, _ref(d, go, torch.float64)):
        torch.testing.assert_close(x, r, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("cfg", ["msda_detr", "msda_tsa", "msda_sca"])
def test_configs_full_size(cfg, dtype):
    d = inputs.msda_inputs(cfg)
    go = _grad_output(d)
    gv, gl, ga = _run(d, go, dtype)
    nq = d["sampling_loc"].shape[1]
    g = torch.Generator().manual_seed(321)
    q_idx = torch.randperm(nq, generator=g)[:300].sort().values
    q_idx = torch.cat([q_idx, torch.tensor([0, nq - 1])]).unique()
    _, rl, ra = _ref(d, go, dtype, q_idx)
    check(gl[:, q_idx], rl, dtype, f"{cfg} full {dtype} grad_sampling_loc")
    check(ga[:, q_idx], ra, dtype, f"{cfg} full {dtype} grad_attn_weight")
    # whole-tensor identities, float64 sums of the kernel's own outputs
    v = d["value"].to(dtype).double()
    a = d["attn_weight"].to(dtype).double()
    out = _api().ms_deform_attn_forward(**_dev(d, dtype)).cpu().double()
    lhs = (go.to(dtype).double() * out).sum().item()
    rel = 1e-4 if dtype == torch.float32 else 2e-2
    scale = (go.to(dtype).double() * out).abs().sum().item()
    assert abs((gv.double() * v).sum().item() - lhs) <= rel * scale, cfg
    assert abs((ga.double() * a).sum().item() - lhs) <= rel * scale, cfg
    for t in (gv, gl, ga):
        assert torch.isfinite(t).all()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_strided_grad_output(dtype):
    """grad_output read through its strides (binding_musa.mu:446-447 views it)."""
    d = inputs.msda_inputs("msda_detr", scale_q=0.01, batch=2)
    go = _grad_output(d)
    wide = torch.zeros(go.shape[0], go.shape[1], 2 * go.shape[2])
    wide[..., ::2] = go
    strided = wide.to(dtype).to(DEV)[..., ::2]
    assert not strided.is_contiguous()
    dd = _dev(d, dtype)
    got = _api().ms_deform_attn_backward(**dd, grad_output=strided)
    ref = _api().ms_deform_attn_backward(**dd, grad_output=go.to(dtype).to(DEV))
    torch.cuda.synchronize()
    for x, r in zip(got, ref):
        check(x.cpu(), r.cpu().double(), dtype, "strided grad_output")


def test_grad_value_accumulates_fp32_and_is_written_fp16():
    """fp32: the kernels add into the caller's grad_value; fp16: the fp32 accumulator is
    narrowed over it (binding_musa.mu:508-510)."""
    import _modulated_deform_conv_ext as ext
    d = inputs.msda_inputs("msda_sca", scale_q=0.005, batch=1)
    go = _grad_output(d)
    for dtype in (torch.float32, torch.float16):
        dd = _dev(d, dtype)
        gv = torch.full_like(dd["value"], 3.0)
        gl = torch.full_like(dd["sampling_loc"], 7.0)
        ga = torch.full_like(dd["attn_weight"], 7.0)
        ext.backward(dd["value"], dd["spatial_shapes"], dd["level_start_index"],
                     dd["sampling_loc"], dd["attn_weight"], go.to(dtype).to(DEV), gv, gl, ga)
        torch.cuda.synchronize()
        rv, rl, ra = _ref(d, go, dtype)
        base = 3.0 if dtype == torch.float32 else 0.0
        check(gv.cpu(), rv + base, dtype, f"{dtype} grad_value")
        check(gl.cpu(), rl, dtype, f"{dtype} grad_sampling_loc written")
        check(ga.cpu(), ra, dtype, f"{dtype} grad_attn_weight written")


@pytest.mark.parametrize("geom", [
    (2, [(5, 6), (3, 4)], 7, 2, 48, 3),        # D not a power of two
    (1, [(4, 7)], 5, 3, 96, 2),                # D > 64: two channel passes
    (2, [(1, 1), (2, 3), (6, 2)], 9, 4, 8, 5),
    (1, [(9, 11)], 13, 1, 1, 1),
    (3, [(3, 3), (2, 2)], 6, 2, 64, 4),
    (2, [(1, 1), (7, 3), (5, 9)], 11, 3, 32, 5),  # D = 32 kernel, ragged levels
])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16,
                                   torch.float64], ids=IDS + ["fp64"])
def test_generic_shapes(geom, dtype):
    d = inputs.msda_random(*geom, seed=13, loc_lo=-0.3, loc_hi=1.3)
    go = _grad_output(d, seed=3)
    got = _run(d, go, dtype)
    ref = _ref(d, go, dtype)
    if dtype == torch.float64:
        for x, r in zip(got, ref):
            torch.testing.assert_close(x, r, rtol=1e-10, atol=1e-10)
    else:
        _check3(got, ref, dtype, f"{geom} {dtype}")


def _grid_queries(batch, H, W, heads, points, jitter_px, far_frac, seed):
    """One level, one query per cell (q = y*W + x) sampling around its cell centre with
    `jitter_px` pixels of Gaussian noise; a `far_frac` share of the samples is moved to a
    random place in [-0.2, 1.2]^2 (far from its query, some outside the window)."""
    g = torch.Generator().manual_seed(seed)
    spatial_shapes, lsi, s = inputs.msda_meta([(H, W)])
    value = torch.randn(batch, s, heads, 32, generator=g)
    q = torch.arange(s)
    ctr = torch.stack([((q % W).double() + 0.5) / W, ((q // W).double() + 0.5) / H], -1)
    shape = (batch, s, heads, 1, points, 2)
    loc = ctr.float().view(1, s, 1, 1, 1, 2).expand(*shape).clone()
    loc[..., 0] += jitter_px / W * torch.randn(shape[:-1], generator=g)
    loc[..., 1] += jitter_px / H * torch.randn(shape[:-1], generator=g)
    far = torch.rand(shape[:-1], generator=g) < far_frac
    wild = -0.2 + 1.4 * torch.rand(shape, generator=g)
    loc = torch.where(far.unsqueeze(-1), wild, loc)
    attn = torch.softmax(torch.randn(batch, s, heads, points, generator=g), -1)
    return dict(value=value, spatial_shapes=spatial_shapes, level_start_index=lsi,
                sampling_loc=loc, attn_weight=attn.view(batch, s, heads, 1, points))


@pytest.mark.parametrize("geom", [
    # batch, H, W, heads, points, jitter px, far share
    (2, 23, 37, 2, 4, 2.0, 0.05),   # edge tiles on both axes
    (1, 8, 8, 3, 1, 1.0, 0.0),      # one tile exactly, one point
    (1, 9, 17, 1, 3, 3.0, 0.1),
    (2, 40, 30, 2, 2, 4.0, 0.02),   # wide jitter: many samples beyond the owner margin
])
@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_grid_queries(geom, dtype):
    """Queries on the grid cells of a one-level map (the temporal self-attention form),
    through the sorted path (the API's workspace) and through the owner kernels (a
    workspace without the sorted path's buffers: grad_value from the per-position owner
    pass plus atomics for the samples far from their query); all three gradients are
    compared whole with the oracle."""
    d = _grid_queries(*geom, seed=sum(geom[:5]))
    go = _grad_output(d, seed=5)
    ref = _ref(d, go, dtype)
    _check3(_run(d, go, dtype), ref, dtype, f"grid {geom} {dtype} sorted path")
    _check3(_run_workspace(d, go, dtype, _accumulator_bytes(d, dtype)), ref, dtype,
            f"grid {geom} {dtype} owner kernels")


def _crowded_grid(H, W, heads, cy, cx, seed):
    """Queries on the cells of an H x W map whose 4 samples move up to 5 cells towards
    cell (cy, cx) (so every sample stays within the owner margin of its query): the 8 x 8
    tile holding (cy, cx) receives several thousand corner pairs."""
    g = torch.Generator().manual_seed(seed)
    spatial_shapes, lsi, s = inputs.msda_meta([(H, W)])
    value = torch.randn(1, s, heads, 32, generator=g)
    q = torch.arange(s)
    qy, qx = (q // W).double(), (q % W).double()
    ty = qy + (cy - qy).clamp(-5, 5)
    tx = qx + (cx - qx).clamp(-5, 5)
    shape = (1, s, heads, 1, 4)
    jy = ty.view(1, s, 1, 1, 1) + 0.5 + 0.3 * torch.randn(shape, generator=g, dtype=torch.float64)
    jx = tx.view(1, s, 1, 1, 1) + 0.5 + 0.3 * torch.randn(shape, generator=g, dtype=torch.float64)
    # keep every corner within 5 cells of its query (the jitter must not push it out)
    jy = torch.minimum(torch.maximum(jy, qy.view(1, s, 1, 1, 1) - 4.4), qy.view(1, s, 1, 1, 1) + 5.4)
    jx = torch.minimum(torch.maximum(jx, qx.view(1, s, 1, 1, 1) - 4.4), qx.view(1, s, 1, 1, 1) + 5.4)
    loc = torch.stack([jx / W, jy / H], -1).float()
    attn = torch.softmax(torch.randn(1, s, heads, 4, generator=g), -1)
    d = dict(value=value, spatial_shapes=spatial_shapes, level_start_index=lsi,
             sampling_loc=loc, attn_weight=attn.view(1, s, heads, 1, 4))
    # corner pairs landing in the crowded tile (h_im = loc * H - 0.5, as the kernels)
    hi = (loc[..., 1].double() * H - 0.5).floor()
    wi = (loc[..., 0].double() * W - 0.5).floor()
    t0y, t0x = cy // 8 * 8, cx // 8 * 8
    n = 0
    for dy in (0, 1):
        for dx in (0, 1):
            yy, xx = hi + dy, wi + dx
            n += int(((yy >= t0y) & (yy < t0y + 8) & (xx >= t0x) & (xx < t0x + 8)).sum() // heads)
    return d, n


def test_grid_queries_accumulate_fp32():
    """Grid queries, fp32: grad_value is added to what the caller holds (here 3.0
    everywhere), including in a crowded tile, by the sorted path (API) and by the owner
    kernels (no workspace)."""
    import _modulated_deform_conv_ext as ext
    for d in (_grid_queries(1, 19, 21, 2, 4, 2.0, 0.05, seed=8), _crowded_grid(30, 28, 2, 12, 13, seed=4)[0]):
        go = _grad_output(d, seed=7)
        dd = _dev(d, torch.float32)
        gv = torch.full_like(dd["value"], 3.0)
        gl = torch.empty_like(dd["sampling_loc"])
        ga = torch.empty_like(dd["attn_weight"])
        ext.backward(dd["value"], dd["spatial_shapes"], dd["level_start_index"],
                     dd["sampling_loc"], dd["attn_weight"], go.to(DEV), gv, gl, ga)
        torch.cuda.synchronize()
        rv, rl, ra = _ref(d, go, torch.float32)
        for what, got in (("sorted path", (gv.cpu(), gl.cpu(), ga.cpu())),
                          ("owner kernels", _run_workspace(d, go, torch.float32, 0, gv_init=3.0))):
            check(got[0], rv + 3.0, torch.float32, f"grid grad_value accumulated, {what}")
            check(got[1], rl, torch.float32, f"grid grad_sampling_loc, {what}")
            check(got[2], ra, torch.float32, f"grid grad_attn_weight, {what}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_grid_queries_crowded_tile(dtype):
    """Owner kernels (a workspace without the sorted path's buffers): a tile with more
    corner pairs than the owner pass keeps in LDS (2560) takes the atomic branch; the
    result still matches the oracle. The sorted path is checked on the same inputs."""
    d, pairs = _crowded_grid(30, 28, 2, 12, 13, seed=4)
    assert pairs > 2560, pairs
    go = _grad_output(d, seed=6)
    ref = _ref(d, go, dtype)
    _check3(_run_workspace(d, go, dtype, _accumulator_bytes(d, dtype)), ref, dtype,
            f"crowded {dtype} owner kernels")
    _check3(_run(d, go, dtype), ref, dtype, f"crowded {dtype} sorted path")


# Coarse-level backward constants (msda_bwd.hip): a workgroup takes COARSE_Q queries of
# one (batch, head) slice and keeps at most COARSE_CAP corner pairs in LDS.
COARSE_Q, COARSE_CAP = 256, 16384


def _valid_corners(loc, shapes):
    """Corners inside their level of the samples in loc [..., L, P, 2] (h_im = y*H - 0.5,
    the window gate, then per-corner bounds), counted as the kernels count pairs."""
    Hs = shapes[:, 0].double().view(-1, 1)
    Ws = shapes[:, 1].double().view(-1, 1)
    him = loc[..., 1].double() * Hs - 0.5
    wim = loc[..., 0].double() * Ws - 0.5
    inside = (him > -1) & (wim > -1) & (him < Hs) & (wim < Ws)
    hl, wl = him.floor(), wim.floor()
    n = 0
    for dy in (0, 1):
        for dx in (0, 1):
            y, x = hl + dy, wl + dx
            n += int((inside & (y >= 0) & (y < Hs) & (x >= 0) & (x < Ws)).sum())
    return n


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_coarse_levels_overflow(dtype):
    """Atomic kernels (a workspace without the sorted path's buffers). Small levels only
    (all of them "coarse": 96 positions), 8 points per level and D = 32: the first
    workgroup's COARSE_Q queries bring more valid corner pairs than its LDS list holds
    (COARSE_CAP), so it adds them one by one; the result matches the oracle. The sorted
    path (full workspace) is checked on the same inputs."""
    d = inputs.msda_random(1, [(6, 7), (4, 5), (3, 3), (2, 2)], 300, 2, 32, 8, seed=21,
                           loc_lo=0.05, loc_hi=0.95)
    first = d["sampling_loc"][0, :COARSE_Q, 0]  # the first workgroup: batch 0, head 0
    pairs = _valid_corners(first, d["spatial_shapes"])
    assert pairs > COARSE_CAP, pairs
    go = _grad_output(d, seed=9)
    ref = _ref(d, go, dtype)
    _check3(_run_workspace(d, go, dtype, _accumulator_bytes(d, dtype)), ref, dtype,
            f"coarse overflow, atomic kernels {dtype}")
    _check3(_run(d, go, dtype), ref, dtype, f"coarse overflow, sorted path {dtype}")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("cfg", ["msda_detr", "msda_sca"])
def test_atomic_kernels_reduced(cfg, dtype):
    """The D = 32 atomic kernels (workspace below the sorted path's size) on the reduced
    BASELINE configurations, whole."""
    d = inputs.msda_inputs(cfg, scale_q=0.02, batch=1)
    go = _grad_output(d)
    _check3(_run_workspace(d, go, dtype, _accumulator_bytes(d, dtype)), _ref(d, go, dtype),
            dtype, f"{cfg} atomic kernels {dtype}")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_sorted_concentrated(dtype):
    """Sorted path with every sample near one point: each slice's corners fall in a few
    positions of one 256-position bucket per level (24 K corners: six accumulate chunks
    that add with atomics), and single positions take thousands of corners (one lane group
    walks them all)."""
    g = torch.Generator().manual_seed(31)
    d = inputs.msda_random(1, [(16, 16), (8, 8)], 1500, 2, 32, 4, seed=31)
    d["sampling_loc"] = 0.5 + 0.02 * torch.randn(d["sampling_loc"].shape, generator=g)
    go = _grad_output(d, seed=5)
    _check3(_run(d, go, dtype), _ref(d, go, dtype), dtype, f"concentrated {dtype}")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_sorted_ragged(dtype):
    """Sorted path with 12 (batch, head) slices (not a multiple of the 8 XCD lists), a
    spatial size of 790 (the last 256-position bucket partial), 333 queries (not a
    multiple of a place block's 85) and samples outside the window."""
    d = inputs.msda_random(3, [(20, 30), (10, 15), (5, 8)], 333, 4, 32, 4, seed=17,
                           loc_lo=-0.2, loc_hi=1.2)
    go = _grad_output(d, seed=8)
    _check3(_run(d, go, dtype), _ref(d, go, dtype), dtype, f"ragged {dtype}")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("num_query", [60, 2500], ids=["one_chunk", "pieces"])
def test_sorted_bucket_edges(num_query, dtype):
    """Sorted path, records at the edges of the 256-position buckets of a 6 x 100 map
    (S = 600: buckets 0-255, 256-511 and a partial 512-599). The five points of every
    query sit (with 0.04 px of jitter) in five cells:
      A (2.4, 55.3): the top pair at positions 255 / 256 crosses from bucket 0 into 1;
      B (4.6, 11.7): the bottom pair at 511 / 512 crosses into the partial bucket;
      C (1.5, -0.4): the left corners outside the map (right-only records at 100, 200);
      D (0.2, 99.3): the right corners outside (left-only records at 99, 199, next to C's);
      E (5.5, 30.5): the bottom row outside (one record, in the partial bucket).
    60 queries: every bucket is one accumulate chunk (read-modify-write, the first and the
    extra row with atomics); 2,500: buckets of several chunks and pieces (atomics)."""
    H, W, P = 6, 100, 5
    cells = torch.tensor([[2.4, 55.3], [4.6, 11.7], [1.5, -0.4], [0.2, 99.3], [5.5, 30.5]],
                         dtype=torch.float64)
    g = torch.Generator().manual_seed(41)
    B, NH = 1, 2
    him = cells[:, 0] + 0.04 * (2 * torch.rand(B, num_query, NH, 1, P, generator=g) - 1)
    wim = cells[:, 1] + 0.04 * (2 * torch.rand(B, num_query, NH, 1, P, generator=g) - 1)
    loc = torch.stack([(wim + 0.5) / W, (him + 0.5) / H], -1).float()
    # the corner cells the kernels see (h_im = loc * H - 0.5 in fp32)
    for t in (torch.float32, torch.float16, torch.bfloat16):
        lt = loc.to(t).float()
        hh, ww = lt[..., 1] * H - 0.5, lt[..., 0] * W - 0.5
        assert torch.equal(hh.floor()[0, :, :, 0], cells[:, 0].floor().float().expand(num_query, NH, P))
        assert torch.equal(ww.floor()[0, :, :, 0], cells[:, 1].floor().float().expand(num_query, NH, P))
    d = dict(value=torch.randn(B, H * W, NH, 32, generator=g),
             spatial_shapes=torch.tensor([[H, W]], dtype=torch.int64),
             level_start_index=torch.tensor([0], dtype=torch.int64),
             sampling_loc=loc.contiguous(),
             attn_weight=torch.softmax(torch.randn(B, num_query, NH, P, generator=g), -1)
             .view(B, num_query, NH, 1, P).contiguous())
    go = _grad_output(d, seed=12)
    _check3(_run(d, go, dtype), _ref(d, go, dtype), dtype, f"bucket edges {num_query} {dtype}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_sorted_unaligned_grad_value(dtype):
    """16-bit sorted path with grad_value 2 bytes past an 8-byte boundary (a contiguous view
    one element into a larger buffer): the workspace clear and the narrowing run as their
    own passes instead of inside the count and coordinate kernels. Same gradients as the
    aligned call, and the elements around grad_value keep their values."""
    import _bevk as b
    d = inputs.msda_random(2, [(20, 30), (10, 15)], 300, 4, 32, 4, seed=23)
    go = _grad_output(d, seed=9)
    dd = _dev(d, dtype)
    value, loc = dd["value"], dd["sampling_loc"]
    B, S, NH, D = value.shape
    Lq, L, P = loc.shape[1], loc.shape[3], loc.shape[4]
    g4 = go.to(dtype).to(DEV).view(B, Lq, NH, D)
    ws_bytes = b.lib().bevk_msda_backward_workspace_bytes(b.dtype_code(value), B, S, NH, D, L,
                                                          Lq, P)
    n = value.numel()
    outs = []
    for shift in (0, 1):
        buf = torch.full((n + 8,), 3.0, dtype=dtype, device=DEV)
        gv = buf[shift:shift + n].view(value.shape)
        assert gv.data_ptr() % 8 == 2 * shift
        gl = torch.empty_like(loc)
        ga = torch.empty_like(dd["attn_weight"])
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
        b.call("bevk_msda_backward", b.dtype_code(value), b.ptr(value),
               b.ptr(dd["spatial_shapes"]), b.ptr(dd["level_start_index"]), b.ptr(loc),
               b.ptr(dd["attn_weight"]), b.ptr(g4), *g4.stride(), B, S, NH, D, L, Lq, P, 64, 0,
               b.ptr(gv), b.ptr(gl), b.ptr(ga), b.ptr(ws), ws_bytes, b.stream_of(value))
        torch.cuda.synchronize()
        outs.append((gv.cpu().float(), gl.cpu().float(), ga.cpu().float(), buf.cpu()))
    (gv0, gl0, ga0, _), (gv1, gl1, ga1, buf1) = outs
    for name, x, r in (("grad_value", gv1, gv0), ("grad_sampling_loc", gl1, gl0),
                       ("grad_attn_weight", ga1, ga0)):
        check(x, r, dtype, f"unaligned grad_value run, {name} vs aligned")
    assert buf1[0].item() == 3.0 and bool((buf1[n + 1:] == 3.0).all())
    ref = _ref(d, go, dtype)
    check(gv1, ref[0], dtype, "unaligned grad_value vs oracle")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
@pytest.mark.parametrize("case", ["hw_below_s", "level_offset"])
def test_one_level_not_a_grid(case, dtype):
    """One level with num_query == spatial_size whose shapes do not make the queries its
    cells: H*W < S (the positions past H*W are never sampled), or the level starting at
    position 16. The grid-query owner pass must not take them (both owner kernels read
    the device metadata and fall back to atomics for every sample); through the owner
    kernels and the sorted path every gradient matches the oracle and the unsampled
    positions of grad_value are zero."""
    H, W, S = 9, 11, 120
    lsi0 = 0 if case == "hw_below_s" else 16
    g = torch.Generator().manual_seed(5)
    d = dict(value=torch.randn(2, S, 2, 32, generator=g),
             spatial_shapes=torch.tensor([[H, W]], dtype=torch.int64),
             level_start_index=torch.tensor([lsi0], dtype=torch.int64),
             sampling_loc=-0.1 + 1.2 * torch.rand(2, S, 2, 1, 4, 2, generator=g),
             attn_weight=torch.softmax(torch.randn(2, S, 2, 4, generator=g), -1).view(2, S, 2, 1, 4))
    go = _grad_output(d, seed=8)
    ref = _ref(d, go, dtype)
    unsampled = torch.ones(S, dtype=torch.bool)
    unsampled[lsi0:lsi0 + H * W] = False
    for what, got in (("owner kernels", _run_workspace(d, go, dtype, _accumulator_bytes(d, dtype))),
                      ("sorted path", _run(d, go, dtype))):
        _check3(got, ref, dtype, f"one level {case} {dtype} {what}")
        assert got[0][:, unsampled].abs().max().item() == 0.0, what


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
@pytest.mark.parametrize("cfg", ["msda_detr", "msda_tsa", "msda_sca"])
def test_force_generic_col2im_full_size(cfg, dtype):
    """force_generic_col2im selects the per-unit atomic kernel for every level (the
    reference's generic col2im). At full BASELINE size its three gradients are compared
    elementwise with the default path (D = 32 kernel, coarse-level sort, grid owner
    pass): two independent implementations of every grad_value element."""
    d = inputs.msda_inputs(cfg)
    go = _grad_output(d)
    dd = _dev(d, dtype)
    gd = go.to(dtype).to(DEV)
    fast = _api().ms_deform_attn_backward(**dd, grad_output=gd)
    generic = _api().ms_deform_attn_backward(**dd, grad_output=gd, force_generic_col2im=True)
    torch.cuda.synchronize()
    for name, a, r in zip(("grad_value", "grad_sampling_loc", "grad_attn_weight"), fast, generic):
        a, r = a.double().cpu(), r.double().cpu()
        if dtype == torch.float32:
            # two fp32 results: grad_value and grad_attn_weight agree within twice the
            # elementwise bound. grad_sampling_loc is W * a * (S2 - S1 ...), a scaled
            # difference of 32-term corner sums: each kernel's fp32 summation error (a few
            # 1e-6 of S) is multiplied by W * a (up to 50 at 200 x 200), so it is bounded
            # against the tensor's own scale (mean |r| ~ 1e2 here), the SURVEY appendix A.3
            # norm, at 2e-4.
            err = (a - r).abs()
            if name == "grad_sampling_loc":
                bad = err > 2e-4 * (r.abs() + r.abs().mean())
            else:
                bad = err > 2e-4 + 2e-4 * r.abs()
            assert not bad.any(), (f"{cfg} {name}: {int(bad.sum())}/{a.numel()} outside "
                                   f"2e-4 abs+rel, max err {err.max().item():.3e}")
        else:
            check(a, r, dtype, f"{cfg} {dtype} {name} default vs generic")


@pytest.mark.parametrize("num_query,heads", [((1 << 21) + 5, 8), ((1 << 22) + 3, 1)])
def test_large_unit_counts(num_query, heads):
    """Unit decoding at scale. The D = 32 kernel decodes (batch, query, head) from its unit
    index with float reciprocals and one correction step, exact while batch x queries
    < 2^22 (its launch bound): 8 heads x (2^21 + 5) queries put the unit index past 2^24,
    where its float conversion rounds. 2^22 + 3 queries are past the bound and take the
    general kernel. grad_sampling_loc / grad_attn_weight of queries spread over the range
    (each depends on its own query and head only) against the oracle on that subset."""
    d = inputs.msda_random(1, [(3, 5), (2, 2)], num_query, heads, 32, 1, seed=21,
                           loc_lo=-0.3, loc_hi=1.3)
    g = torch.Generator().manual_seed(4)
    q_idx = torch.cat([torch.arange(16), torch.arange(num_query - 16, num_query),
                       torch.randint(16, num_query - 16, (32,), generator=g)]).unique()
    gen = torch.Generator(device=DEV).manual_seed(9)
    go = torch.randn(1, num_query, heads * 32, generator=gen, device=DEV).half()
    dd = _dev(d, torch.float16)
    _, gl, ga = _api().ms_deform_attn_backward(**dd, grad_output=go)
    torch.cuda.synchronize()
    sub = dict(d, sampling_loc=d["sampling_loc"][:, q_idx], attn_weight=d["attn_weight"][:, q_idx])
    go_sub = go[:, q_idx.to(DEV)].float().cpu()
    del go, dd
    _, rl, ra = _ref(sub, go_sub, torch.float16)
    check(gl[:, q_idx.to(DEV)].cpu(), rl, torch.float16, f"{num_query}x{heads} grad_sampling_loc")
    check(ga[:, q_idx.to(DEV)].cpu(), ra, torch.float16, f"{num_query}x{heads} grad_attn_weight")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_empty_queries(dtype):
    d = inputs.msda_random(2, [(3, 4)], 0, 2, 32, 2)
    go = torch.zeros(2, 0, 64)
    gv, gl, ga = _run(d, go, dtype)
    assert gl.numel() == 0 and ga.numel() == 0
    assert gv.abs().max().item() == 0.0


def test_im2col_step_contract():
    d = inputs.msda_random(6, [(3, 4)], 2, 2, 32, 2)
    go = _grad_output(d)
    with pytest.raises(RuntimeError, match="batch must divide im2col_step"):
        _run(d, go, torch.float32, im2col_step=4)
    got = _run(d, go, torch.float32, im2col_step=3)
    _check3(got, _ref(d, go, torch.float32), torch.float32, "im2col_step=3")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_autograd_function(dtype):
    """MultiScaleDeformableAttnFunction: autograd gradients equal the oracle's; the
    integer inputs get none."""
    d = inputs.msda_inputs("msda_sca", scale_q=0.005, batch=2)
    go = _grad_output(d)
    dd = _dev(d, dtype)
    v = dd["value"].requires_grad_(True)
    loc = dd["sampling_loc"].requires_grad_(True)
    a = dd["attn_weight"].requires_grad_(True)
    out = _api().multi_scale_deformable_attn(v, dd["spatial_shapes"], dd["level_start_index"],
                                             loc, a)
    (out * go.to(dtype).to(DEV)).sum().backward()
    torch.cuda.synchronize()
    _check3((v.grad.cpu(), loc.grad.cpu(), a.grad.cpu()), _ref(d, go, dtype), dtype,
            f"Function {dtype}")


def test_autograd_expanded_grad_output():
    """A gradient that cannot be viewed per (b, q, head, c) (an expanded one) is made dense."""
    d = inputs.msda_random(1, [(4, 5)], 3, 2, 8, 2, seed=2)
    dd = _dev(d, torch.float32)
    v = dd["value"].requires_grad_(True)
    out = _api().multi_scale_deformable_attn(v, dd["spatial_shapes"], dd["level_start_index"],
                                             dd["sampling_loc"], dd["attn_weight"])
    out.sum().backward()                       # grad_output = ones expanded from a scalar
    torch.cuda.synchronize()
    go = torch.ones(1, 3, 16)
    rv, _, _ = _ref(d, go, torch.float32)
    check(v.grad.cpu(), rv, torch.float32, "expanded grad_output")


def test_gradcheck_fp64():
    """Finite differences of the GPU forward against the GPU backward, float64, locations
    away from the integer grid lines."""
    d = inputs.msda_random(1, [(3, 4), (2, 3)], 3, 2, 4, 2, seed=21, loc_lo=-0.2,
                           loc_hi=1.2)
    dd = _dev(d, torch.float64)
    fn = _api().MultiScaleDeformableAttnFunction.apply
    torch.autograd.gradcheck(
        lambda v, loc, a: fn(v, dd["spatial_shapes"], dd["level_start_index"], loc, a, 64),
        (dd["value"].requires_grad_(True), dd["sampling_loc"].requires_grad_(True),
         dd["attn_weight"].requires_grad_(True)), eps=1e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["fp32", "fp16"])
def test_backward_workspace_cap(dtype, monkeypatch):
    """ms_deform_attn_backward with the sorted path's workspace (no cap) and with
    max_workspace_bytes=0 (the atomic kernels with the reference's memory use: nothing for
    fp32, the fp32 grad_value accumulator for fp16), and with the cap from
    BEVK_MSDA_BACKWARD_MAX_WORKSPACE: all three against the oracle; the capped calls'
    peak device memory is below the uncapped call's by about the sorted buffers."""
    import _modulated_deform_conv_ext as ext
    monkeypatch.delenv(ext.MSDA_BACKWARD_MAX_WORKSPACE_ENV, raising=False)
    d = inputs.msda_inputs("msda_sca", scale_q=0.05)
    go = _grad_output(d)
    ref = _ref(d, go, dtype)
    value = d["value"].to(dtype)
    L, Q, P = d["sampling_loc"].shape[3], d["sampling_loc"].shape[1], d["sampling_loc"].shape[4]
    full, least = ext.backward_workspace_bytes(value, L, Q, P)
    assert full > least

    def run_peak(**kw):
        dd = _dev(d, dtype)
        g = go.to(dtype).to(DEV)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        got = _api().ms_deform_attn_backward(**dd, grad_output=g, **kw)
        torch.cuda.synchronize()
        return [t.cpu() for t in got], torch.cuda.max_memory_allocated() - base

    got, peak_full = run_peak()
    _check3(got, ref, dtype, "sorted path")
    got, peak_capped = run_peak(max_workspace_bytes=0)
    _check3(got, ref, dtype, "capped")
    monkeypatch.setenv(ext.MSDA_BACKWARD_MAX_WORKSPACE_ENV, str(full - 1))
    got, peak_env = run_peak()
    _check3(got, ref, dtype, "capped from the environment")
    assert peak_full - peak_capped >= 0.9 * (full - least), (peak_full, peak_capped, full, least)
    assert peak_env == peak_capped


def _exact_centre(n):
    """Index i < n - 1 whose pixel centre (i + 0.5) / n is exact in fp32, fp16 and bf16."""
    from fractions import Fraction
    for i in range(n - 1):
        fr = Fraction(2 * i + 1, 2 * n)
        if fr.denominator & (fr.denominator - 1) == 0 and fr.numerator < 256:
            return i, float(fr)
    raise ValueError(f"no exact pixel centre for size {n}")


def _poison_bwd(d, go, seed):
    """Non-finite value / grad_output, following the reference's per-sample gradient
    (ms_deform_attn_kernels.cuh:427-490): every in-bounds corner enters the position and
    attention gradients and receives w * top * a in grad_value, whatever its weight w.
    Units (batch 0, query 0, head 0) and (0, 1, head 1 % NH) sample the exact centre of
    level-0 pixel (y, x) at every point (other levels far outside):
      * value NaN at (y + 1, x + 1) of head 0, a corner of weight 0, the other corners
        finite -> that unit's grad_sampling_loc and grad_attn_weight are NaN;
      * grad_output NaN for the second unit -> grad_value NaN at all four corners of its
        head, the three of weight 0 included;
      * a few random (position, head) rows of value hold NaN or +Inf."""
    g = torch.Generator().manual_seed(seed)
    v, loc = d["value"], d["sampling_loc"]
    B, S, NH, D = v.shape
    shapes = d["spatial_shapes"].tolist()
    starts = d["level_start_index"].tolist()
    for (H, W), start in zip(shapes, starts):
        for b in range(B):
            pos = start + torch.randint(0, H * W, (4,), generator=g)
            heads = torch.randint(0, NH, (4,), generator=g)
            for k in range(4):
                v[b, pos[k], heads[k], :] = float("nan") if k < 2 else float("inf")
    H0, W0 = shapes[0]
    y, ly = _exact_centre(H0)
    x, lx = _exact_centre(W0)
    h1 = 1 % NH
    for q, h in ((0, 0), (1, h1)):
        loc[0, q, h] = -5.0
        loc[0, q, h, 0, :, 0] = lx
        loc[0, q, h, 0, :, 1] = ly
    for p in (y * W0 + x, y * W0 + x + 1, (y + 1) * W0 + x):
        v[0, p, 0, :] = 1.0
    v[0, (y + 1) * W0 + x + 1, 0, :] = float("nan")
    go[0, 1, h1 * D:(h1 + 1) * D] = float("nan")
    return [(y + dy) * W0 + x + dx for dy in (0, 1) for dx in (0, 1)], h1


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("kind", ["sorted", "atomic", "owner", "generic"])
def test_nonfinite_backward(kind, dtype):
    """NaN / Inf in value and grad_output give NaN / Inf in all three gradients exactly where
    the float64 oracle does, through each backward path (the API's sorted path, the D = 32
    atomic kernels, the grid-query owner kernels, the generic kernels for D = 64); finite
    entries match it to tolerance."""
    if kind == "owner":
        d = _grid_queries(1, 23, 37, 2, 4, 2.0, 0.05, seed=61)
    elif kind == "generic":
        d = inputs.msda_random(2, [(6, 8), (3, 5)], 40, 2, 64, 4, seed=62, loc_lo=-0.3,
                               loc_hi=1.3)
    else:
        d = inputs.msda_random(2, [(12, 16), (6, 8), (3, 4), (2, 2)], 300, 4, 32, 8, seed=63,
                               loc_lo=-0.3, loc_hi=1.3)
    go = _grad_output(d, seed=64)
    corners, h1 = _poison_bwd(d, go, seed=65)
    if kind in ("atomic", "owner"):
        got = _run_workspace(d, go, dtype, _accumulator_bytes(d, dtype))
    else:
        got = _run(d, go, dtype)
    ref = _ref(d, go, dtype)
    what = f"nonfinite backward {kind} {dtype}"
    for name, x, r in zip(("grad_value", "grad_sampling_loc", "grad_attn_weight"), got, ref):
        x, r = x.double(), r.double()
        assert torch.equal(torch.isnan(x), torch.isnan(r)), f"{what} {name}: NaN pattern"
        assert torch.equal(torch.isinf(x), torch.isinf(r)), f"{what} {name}: Inf pattern"
        assert torch.equal(x[torch.isinf(r)], r[torch.isinf(r)]), f"{what} {name}: Inf sign"
        fin = torch.isfinite(r)
        check(x[fin], r[fin], dtype, f"{what} {name}")
    gv, gl, ga = got
    assert torch.isnan(gl[0, 0, 0, 0]).all() and torch.isnan(ga[0, 0, 0, 0]).all(), \
        f"{what}: weight-0 NaN corner left out of the position gradient"
    for p in corners:
        assert torch.isnan(gv[0, p, h1].float()).all(), \
            f"{what}: grad_value of a corner of weight 0 missed the NaN grad_output"
    fin = torch.isfinite(ref[1]).double().mean().item()
    assert 0.05 < fin < 0.999, f"{what}: degenerate poison pattern"


@pytest.mark.parametrize("nq", [(1 << 22) - 4, (1 << 22) + 4], ids=["below", "above"])
def test_sorted_path_query_limit(nq):
    """fp16, one head, one 512 x 512 level, one point, about 2^22 queries: the API (the
    sorted path below 2^22 queries, bkt_layout: its record word is query << 8 | position
    in bucket; the atomic kernels from 2^22 on) against the D = 32 atomic kernels through
    the C ABI, every output."""
    import _bevk as bk
    dt = torch.float16
    H = W = 512
    g = torch.Generator(device=DEV).manual_seed(71)
    value = torch.randn(1, H * W, 1, 32, generator=g, device=DEV).to(dt)
    loc = torch.rand(1, nq, 1, 1, 1, 2, generator=g, device=DEV).to(dt)
    attn = torch.rand(1, nq, 1, 1, 1, generator=g, device=DEV).to(dt)
    go = torch.randn(1, nq, 32, generator=g, device=DEV).to(dt)
    shapes = torch.tensor([[H, W]], dtype=torch.int64, device=DEV)
    lsi = torch.zeros(1, dtype=torch.int64, device=DEV)
    api = _api().ms_deform_attn_backward(value, shapes, lsi, loc, attn, grad_output=go)
    gv = torch.zeros_like(value)
    gl = torch.empty_like(loc)
    ga = torch.empty_like(attn)
    ws_bytes = value.numel() * 4  # the fp32 grad_value accumulator only: atomic kernels
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    g4 = go.view(1, nq, 1, 32)
    bk.call("bevk_msda_backward", bk.dtype_code(value), bk.ptr(value), bk.ptr(shapes),
            bk.ptr(lsi), bk.ptr(loc), bk.ptr(attn), bk.ptr(g4), *g4.stride(), 1, H * W, 1, 32,
            1, nq, 1, 64, 0, bk.ptr(gv), bk.ptr(gl), bk.ptr(ga), bk.ptr(ws), ws_bytes,
            bk.stream_of(value))
    torch.cuda.synchronize()
    for name, x, r in zip(("grad_value", "grad_sampling_loc", "grad_attn_weight"), api,
                          (gv, gl, ga)):
        check(x.cpu(), r.cpu(), dt, f"{nq} queries {name}: API vs atomic kernels")
