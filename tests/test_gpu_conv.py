"""ConcordConv2dPackedB on the GPU: the conv is the linear packed path on its
patch matrix (bit-exact against a ConcordLinearPackedB fed the same patches),
and its forward, input gradient and weight gradient match fp32 torch
convolutions of the decoded weight within the north-star tolerance."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from gpu_util import DEV, host, rel_l2, sync

pytestmark = pytest.mark.gpu

CASES = [  # (cin, cout, k, stride, pad, B, H, W)
    (32, 48, 3, 1, 1, 2, 20, 24),
    (64, 40, 3, 2, 1, 2, 17, 15),
    (96, 64, 1, 1, 0, 2, 16, 16),
]


@pytest.fixture(autouse=True)
def _reset_globals():
    from concord_amd import packed_b as pb
    pb.set_ratio_coh(False)
    pb.set_fixed_coh(True)
    pb.set_prototype_semantics(False)
    yield


def _patches(x, k, stride, pad):
    if (k, stride, pad) == (1, 1, 0):
        return x.permute(0, 2, 3, 1).reshape(-1, x.shape[1])
    u = F.unfold(x, (k, k), padding=pad, stride=stride)
    return u.transpose(1, 2).reshape(-1, u.shape[1])


@pytest.mark.parametrize("case", CASES)
def test_conv_is_linear_on_patches_bit_exact(case):
    import concord_amd as ca
    from concord_amd import packed_b as pb
    cin, cout, k, stride, pad, B, H, W = case
    torch.manual_seed(sum(case))
    W0 = torch.randn(cout, cin, k, k) * 0.05
    xs = [torch.randn(B, cin, H, W, device=DEV).to(torch.bfloat16) for _ in range(2)]
    conv = ca.ConcordConv2dPackedB(cin, cout, k, stride=stride, padding=pad, bias=True, device=DEV, lr=2e-3)
    lin = ca.ConcordLinearPackedB(cin * k * k, cout, bias=True, device=DEV, lr=2e-3)
    conv.load_weights(W0)
    lin.load_weights(W0.reshape(cout, -1))
    salt = pb._get_step_counter(DEV)
    for i, x in enumerate(xs):
        xc = x.clone().requires_grad_(True)
        salt.fill_(50 + i)
        y = conv(xc)
        gy = (torch.randn_like(y.float()) * 1e-2).to(torch.bfloat16)
        y.backward(gy)
        conv.rebalance()
        xl = _patches(x, k, stride, pad).contiguous().requires_grad_(True)
        salt.fill_(50 + i)
        yl = lin(xl)
        Ho, Wo = y.shape[2], y.shape[3]
        yl_conv = yl.view(B, Ho * Wo, cout).permute(0, 2, 1).reshape(B, cout, Ho, Wo)
        gyl = gy.reshape(B, cout, Ho * Wo).permute(0, 2, 1).reshape(-1, cout).contiguous()
        yl.backward(gyl)
        lin.rebalance()
        sync()
        np.testing.assert_array_equal(host(y), host(yl_conv))
        np.testing.assert_array_equal(host(conv.packed_w), host(lin.packed_w))
        np.testing.assert_array_equal(host(conv.row_exp), host(lin.row_exp))
        np.testing.assert_array_equal(host(conv.col_exp), host(lin.col_exp))
        np.testing.assert_array_equal(host(conv.v_col), host(lin.v_col))
        np.testing.assert_array_equal(host(conv.bias.grad), host(lin.bias.grad))
        # dx: the adjoint of the patch gather applied to the linear layer's dx
        if (k, stride, pad) == (1, 1, 0):
            dx_ref = xl.grad.view(B, H, W, cin).permute(0, 3, 1, 2)
        else:
            dx_ref = F.fold(xl.grad.view(B, Ho * Wo, -1).transpose(1, 2), (H, W), (k, k),
                            padding=pad, stride=stride)
        np.testing.assert_array_equal(host(xc.grad), host(dx_ref.to(torch.bfloat16)))


@pytest.mark.parametrize("case", CASES)
def test_conv_products_match_fp32(case):
    """y, dx and the weight gradient the update consumes, against fp32 torch
    convolutions of the decoded weight (rel-L2 <= 1e-2)."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    cin, cout, k, stride, pad, B, H, W = case
    torch.manual_seed(100 + sum(case))
    conv = ca.ConcordConv2dPackedB(cin, cout, k, stride=stride, padding=pad, bias=True, device=DEV, lr=1e-3)
    with torch.no_grad():
        conv.bias.copy_((torch.randn(cout) * 0.1).to(torch.bfloat16))
    Wd = conv.weight.detach().float().clone()
    bd = conv.bias.detach().float().clone()
    x = torch.randn(B, cin, H, W, device=DEV).to(torch.bfloat16)
    xc = x.clone().requires_grad_(True)
    cap = []
    pb._DEBUG_CAPTURE = cap
    try:
        y = conv(xc)
        gy = (torch.randn_like(y.float()) * 1e-2).to(torch.bfloat16)
        y.backward(gy)
    finally:
        pb._DEBUG_CAPTURE = None
    sync()
    xf = x.float().requires_grad_(True)
    yf = F.conv2d(xf, Wd, bd, stride=stride, padding=pad)
    yf.backward(gy.float())
    gw = torch.nn.grad.conv2d_weight(x.float(), Wd.shape, gy.float(), stride=stride, padding=pad)
    assert y.shape == yf.shape
    assert rel_l2(host(y.float()), host(yf)) < 1e-2
    assert rel_l2(host(xc.grad.float()), host(xf.grad)) < 1e-2
    assert rel_l2(host(cap[0].float()), host(gw.reshape(cout, -1))) < 1e-2
    assert rel_l2(host(conv.bias.grad.float()), host(gy.float().sum(dim=(0, 2, 3)))) < 1e-2


def test_conv_consolidated_export_shape():
    import concord_amd as ca
    conv = ca.ConcordConv2dPackedB(16, 24, 3, padding=1, device=DEV)
    sd = ca.consolidated_state_dict([conv], ["c"])
    assert sd["c.weight"].shape == (24, 16, 3, 3)
    np.testing.assert_array_equal(host(sd["c.weight"].reshape(24, -1)), host(conv.consolidated_weight()))
    assert conv.weight.shape == (24, 16, 3, 3)


@pytest.mark.parametrize("geom", [  # (B, C, H, W, kh, kw, sh, sw, ph, pw)
    (2, 640, 64, 64, 3, 3, 1, 1, 1, 1),
    (2, 13, 17, 15, 3, 3, 2, 2, 1, 1),     # K = 117: the scalar store path
    (1, 8, 9, 11, 5, 3, 1, 2, 2, 0),       # non-square kernel, mixed stride and padding
    (3, 16, 7, 7, 3, 3, 3, 3, 0, 0),
])
def test_im2col_matches_unfold(geom):
    """The one-pass HIP patch matrix equals torch's unfold + transpose bit for
    bit (a pure gather with zeros outside the image)."""
    from concord_amd import _lib as C
    B, Cin, H, W, kh, kw, sh, sw, ph, pw = geom
    x = torch.randn(B, Cin, H, W, device=DEV).to(torch.bfloat16)
    u = F.unfold(x, (kh, kw), padding=(ph, pw), stride=(sh, sw))
    want = u.transpose(1, 2).reshape(-1, u.shape[1]).contiguous()
    got = torch.empty_like(want)
    C.check(C.lib().concord_conv_im2col(C.ptr(x), B, Cin, H, W, kh, kw, sh, sw, ph, pw, C.ptr(got),
                                        C.stream_of(x.device)), "conv_im2col")
    sync()
    np.testing.assert_array_equal(host(got), host(want))


@pytest.mark.parametrize("geom", [  # (B, C, H, W, kh, kw, sh, sw, ph, pw)
    (2, 640, 64, 64, 3, 3, 1, 1, 1, 1),
    (2, 13, 17, 15, 3, 3, 2, 2, 1, 1),
    (1, 8, 9, 70, 5, 3, 1, 2, 2, 0),
    (3, 16, 7, 7, 3, 3, 3, 3, 0, 0),
    (1, 24, 5, 130, 3, 3, 1, 1, 1, 1),
])
def test_col2im_matches_fp32_fold(oracle, geom):
    """The HIP adjoint of im2col against fold in float64 on the same bf16
    patch gradient: each output is a sum of at most kh * kw terms in fp32
    rounded once to bf16, so it is within half a bf16 ulp (2^-8 relative) of
    the exact sum plus the fp32 accumulation error, which is below
    2^-20 times the sum of the terms' magnitudes."""
    from concord_amd import _lib as C
    B, Cin, H, W, kh, kw, sh, sw, ph, pw = geom
    assert C.lib().concord_conv_col2im_fits(kh, kw, sh, sw)
    Ho, Wo = (H + 2 * ph - kh) // sh + 1, (W + 2 * pw - kw) // sw + 1
    dcols = torch.randn(B * Ho * Wo, Cin * kh * kw, device=DEV).to(torch.bfloat16)
    got = torch.empty((B, Cin, H, W), dtype=torch.bfloat16, device=DEV)
    C.check(C.lib().concord_conv_col2im(C.ptr(dcols), B, Cin, H, W, kh, kw, sh, sw, ph, pw, C.ptr(got),
                                        C.stream_of(got.device)), "conv_col2im")
    sync()
    u = dcols.double().cpu().reshape(B, Ho * Wo, -1).transpose(1, 2)
    exact = F.fold(u, (H, W), (kh, kw), padding=(ph, pw), stride=(sh, sw)).numpy()
    mag = F.fold(u.abs(), (H, W), (kh, kw), padding=(ph, pw), stride=(sh, sw)).numpy()
    g = oracle.bf16_bits_to_f32(host(got)).astype(np.float64)
    tol = 2.0 ** -8 * np.abs(exact) + 2.0 ** -20 * mag
    assert np.all(np.abs(g - exact) <= tol), np.max(np.abs(g - exact) - tol)
