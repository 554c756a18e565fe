"""Host-side behaviour of the Python operator layer on the CPU: device / contiguity /
size checks raise RuntimeError before the library is asked to launch (forward and
backward entry points), the Pack module's backend selection and mmcv checkpoint-key migration
(modulated_deform_conv.py:584-643 of the reference), and BASELINE input generators."""
import pytest
import torch

import _modulated_deform_conv_ext as ext
import modulated_deform_conv as mdc
import msda_opt2
from modulated_deform_conv import modulated_deform_conv as mdc_mod
from oracle import inputs


def test_ext_names_match_reference_binding():
    # the 16 pybind names of csrc/binding.cpp:142-191, plus MSDA forward/backward
    names = {
        "modulated_deformable_im2col_cuda", "modulated_deformable_col2im_cuda",
        "modulated_deformable_im2col_opt_cuda", "modulated_deformable_col2im_opt_cuda",
        "modulated_deformable_col2im_smem_cuda", "modulated_deformable_col2im_coord_cuda",
        "modulated_deformable_col2im_coord_opt_cuda", "modulated_deformable_im2col_nhwc_cuda",
        "modulated_deformable_fused_im2col_nhwc_cuda", "modulated_deformable_col2im_nhwc_cuda",
        "modulated_deformable_col2im_coord_nhwc_cuda",
        "modulated_deformable_gradx_smem_nhwc_cuda",
        "modulated_deformable_gradx_gather_nhwc_cuda",
        "modulated_deformable_col2im_fused_smem_nhwc_cuda",
        "modulated_deformable_col2im_perelem_nhwc_cuda",
        "modulated_deformable_col2im_perelem_smem_nhwc_cuda", "forward", "backward"}
    for n in names:
        assert callable(getattr(ext, n))


def test_cpu_tensors_rejected():
    x = torch.zeros(1, 4, 5, 5)
    off = torch.zeros(1, 18, 5, 5)
    m = torch.zeros(1, 9, 5, 5)
    col = torch.zeros(36, 1, 5, 5)
    with pytest.raises(RuntimeError, match="HIP"):
        ext.modulated_deformable_im2col_opt_cuda(x, off, m, 1, 4, 5, 5, 5, 5, 3, 3, 1, 1, 1, 1,
                                                 1, 1, 1, col)
    with pytest.raises(RuntimeError, match="HIP"):
        mdc.modulated_deform_conv2d(x, off, m, torch.zeros(4, 4, 3, 3), None, 1, 1, 1)
    d = inputs.msda_random(1, [(3, 3)], 2, 8, 32, 4)
    with pytest.raises(RuntimeError, match="HIP device tensor"):
        ext.forward(d["value"], d["spatial_shapes"], d["level_start_index"],
                    d["sampling_loc"], d["attn_weight"])


def test_backward_entry_points_check_their_inputs():
    with pytest.raises(RuntimeError, match="HIP"):
        mdc.ext_modulated_deformable_col2im_smem(torch.zeros(36, 25), torch.zeros(1, 18, 5, 5),
                                                 torch.zeros(1, 9, 5, 5), 1, 4, 5, 5, 3, 3, 1,
                                                 1, 1, 1, 1, 1, 1)
    with pytest.raises(RuntimeError, match="HIP"):
        ext.modulated_deformable_col2im_nhwc_cuda(
            torch.zeros(25, 36), torch.zeros(1, 5, 5, 4), torch.zeros(1, 5, 5, 18),
            torch.zeros(1, 5, 5, 9), 1, 4, 5, 5, 5, 5, 3, 3, 1, 1, 1, 1, 1, 1, 1,
            torch.zeros(1, 5, 5, 4), torch.zeros(1, 5, 5, 18), torch.zeros(1, 5, 5, 9))
    with pytest.raises(RuntimeError, match="deformable_group == 1"):
        ext.modulated_deformable_col2im_nhwc_cuda(*([None] * 18), 2, None, None, None)
    d = inputs.msda_random(1, [(3, 3)], 2, 8, 32, 4)
    go = torch.zeros(1, 2, 256)
    with pytest.raises(RuntimeError, match="HIP device tensor"):
        ext.backward(d["value"], d["spatial_shapes"], d["level_start_index"],
                     d["sampling_loc"], d["attn_weight"], go, torch.zeros_like(d["value"]),
                     torch.zeros_like(d["sampling_loc"]), torch.zeros_like(d["attn_weight"]))


def test_pack_backend_selection(monkeypatch):
    calls = []
    monkeypatch.setattr(mdc_mod, "modulated_deform_conv2d",
                        lambda *a, **k: calls.append("cuda") or torch.zeros(1))
    import modulated_deform_conv.dcn_split_nhwc as dsn
    import modulated_deform_conv.fused_tl as ftl
    monkeypatch.setattr(dsn, "dcn_apply_nchw", lambda *a, **k: calls.append("fuse_c"))
    monkeypatch.setattr(ftl, "dcn_apply_nchw", lambda *a, **k: calls.append("tilelang"))
    x = torch.randn(1, 4, 6, 6)
    monkeypatch.delenv("DCN_BACKEND", raising=False)
    mdc.ModulatedDeformConv2dPack(4, 4, 3, padding=1)(x)
    mdc.ModulatedDeformConv2dPack(4, 4, 3, padding=1, backend="tilelang")(x)
    mdc.ModulatedDeformConv2dPack(4, 4, 3, padding=1, backend="cuda")(x)
    # groups / deform_groups != 1 fall back to the NCHW path
    mdc.ModulatedDeformConv2dPack(4, 4, 3, padding=1, groups=2)(x)
    mdc.ModulatedDeformConv2dPack(4, 4, 3, padding=1, deform_groups=2, backend="tilelang")(x)
    monkeypatch.setenv("DCN_BACKEND", "cuda")
    mdc.ModulatedDeformConv2dPack(4, 4, 3, padding=1)(x)
    assert calls == ["fuse_c", "tilelang", "cuda", "cuda", "cuda", "cuda"]


def test_pack_init_and_checkpoint_migration():
    m = mdc.ModulatedDeformConv2dPack(8, 16, 3, padding=1)
    assert m.conv_offset.weight.shape == (27, 8, 3, 3)
    assert torch.all(m.conv_offset.weight == 0) and torch.all(m.conv_offset.bias == 0)
    bound = 1 / (8 * 9) ** 0.5
    assert m.weight.abs().max() <= bound and torch.all(m.bias == 0)
    # An mmcv v1 checkpoint names the offset conv "<prefix>_offset". Current PyTorch hands a
    # child module only the keys under its own prefix, so (as in the reference) the
    # rename applies when the Pack module itself is the loading root (prefix "").
    from collections import OrderedDict
    sd = OrderedDict((k, v.clone()) for k, v in m.state_dict().items())
    w = torch.randn(27, 8, 3, 3)
    b = torch.randn(27)
    sd.pop("conv_offset.weight")
    sd.pop("conv_offset.bias")
    sd["_offset.weight"] = w
    sd["_offset.bias"] = b
    sd._metadata = OrderedDict({"": {"version": 1}})
    m.load_state_dict(sd)
    assert torch.equal(m.conv_offset.weight, w)
    assert torch.equal(m.conv_offset.bias, b)
    # version 2 checkpoints are loaded as they are
    sd2 = OrderedDict((k, v.clone()) for k, v in m.state_dict().items())
    sd2._metadata = OrderedDict({"": {"version": 2}})
    m.load_state_dict(sd2)


def test_msda_api_requires_device(monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    d = inputs.msda_random(1, [(3, 3)], 2, 8, 32, 4)
    with pytest.raises(RuntimeError, match="requires a HIP device"):
        msda_opt2.ms_deform_attn_forward(**d)
    import msda_musa_opt2
    assert msda_musa_opt2.ms_deform_attn_forward is msda_opt2.ms_deform_attn_forward


def test_baseline_input_generators():
    d = inputs.msda_inputs("msda_sca", scale_q=0.05)
    assert d["level_start_index"].tolist() == [0, 23200, 29000, 30450]
    assert d["value"].shape == (6, 30825, 8, 32)
    loc = d["sampling_loc"]
    outside = ((loc < 0) | (loc > 1)).float().mean().item()
    assert 0.08 < outside < 0.09          # 30% drawn from U[-0.2, 1.2): 2/7 of them outside
    a = d["attn_weight"].sum((-2, -1))
    torch.testing.assert_close(a, torch.ones_like(a))
    d = inputs.msda_inputs("msda_detr", scale_q=0.01)
    assert d["level_start_index"].tolist() == [0, 15000, 18750, 19700]
    assert d["value"].shape[1] == 19947
    d = inputs.msda_inputs("msda_tsa", scale_q=0.01)
    q = torch.arange(d["sampling_loc"].shape[1])
    ref = torch.stack([(q % 200 + 0.5) / 200, (q // 200 + 0.5) / 200], -1).float()
    dev = (d["sampling_loc"] - ref.view(1, -1, 1, 1, 1, 2)).std().item()
    assert 0.009 < dev < 0.011
    c = inputs.dcn_inputs("dcn_res4", batch=1)
    assert c["x"].shape == (1, 256, 58, 100) and c["offset"].shape == (1, 18, 58, 100)
    assert abs(c["weight"].std().item() - (2 / 2304) ** 0.5) < 2e-3


def test_msda_backward_workspace_cap(monkeypatch):
    """The backward's scratch choice (host logic, no launch): the sorted path's workspace
    without a cap; above max_workspace_bytes or BEVK_MSDA_BACKWARD_MAX_WORKSPACE only the
    least the library runs with (nothing for fp32, the fp32 grad_value accumulator for
    16-bit types, as binding_musa.mu:456-467 allocates)."""
    monkeypatch.delenv(ext.MSDA_BACKWARD_MAX_WORKSPACE_ENV, raising=False)
    B, S, NH, D, L, Q, P = 6, 30825, 8, 32, 4, 10000, 8
    for dtype, least in ((torch.float32, 0), (torch.float16, B * S * NH * D * 4),
                         (torch.bfloat16, B * S * NH * D * 4)):
        value = torch.empty(B, S, NH, D, dtype=dtype, device="meta")
        full, lo = ext.backward_workspace_bytes(value, L, Q, P)
        assert lo == least and full > least
        assert ext.backward_workspace_bytes(value, L, Q, P, max_workspace_bytes=full) == (full, lo)
        assert ext.backward_workspace_bytes(value, L, Q, P, max_workspace_bytes=full - 1) == (lo, lo)
        assert ext.backward_workspace_bytes(value, L, Q, P, max_workspace_bytes=0) == (lo, lo)
        monkeypatch.setenv(ext.MSDA_BACKWARD_MAX_WORKSPACE_ENV, str(full - 1))
        assert ext.backward_workspace_bytes(value, L, Q, P) == (lo, lo)
        # the argument wins over the environment
        assert ext.backward_workspace_bytes(value, L, Q, P, max_workspace_bytes=full) == (full, lo)
        monkeypatch.setenv(ext.MSDA_BACKWARD_MAX_WORKSPACE_ENV, "lots")
        with pytest.raises(RuntimeError, match="byte count"):
            ext.backward_workspace_bytes(value, L, Q, P)
        monkeypatch.delenv(ext.MSDA_BACKWARD_MAX_WORKSPACE_ENV)
    # SCA sizes the notes quote: about 370 MB fp32 and 560 MB fp16 for the sorted path
    f32 = ext.backward_workspace_bytes(torch.empty(B, S, NH, D, device="meta"), L, Q, P)[0]
    f16 = ext.backward_workspace_bytes(
        torch.empty(B, S, NH, D, dtype=torch.float16, device="meta"), L, Q, P)[0]
    assert 300e6 < f32 < 450e6 and 450e6 < f16 < 650e6
