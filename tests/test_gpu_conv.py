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


@pytest.mark.parametrize("geom", [  # (B, C, H, W, kh, kw, sh, sw, ph, pw)
    (1, 3, 20, 18, 15, 15, 1, 1, 7, 7),
    (2, 2, 13, 16, 14, 14, 2, 2, 6, 6),
])
def test_col2im_direct_matches_fp32_fold(oracle, geom):
    """Windows too large for the staged col2im tile (more than 192 taps)
    take the unstaged gather (col2im_direct_kernel): the same fixed-order
    fp32 sum, so the same bound against float64 fold as above."""
    from concord_amd import _lib as C
    B, Cin, H, W, kh, kw, sh, sw, ph, pw = geom
    assert C.lib().concord_conv_col2im_fits(kh, kw, sh, sw) == 0
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


@pytest.mark.parametrize("case", [(64, 64, 3, 1, 1, 2, 12, 10), (96, 64, 1, 1, 0, 2, 8, 8),
                                  (8, 16, 3, 1, 1, 1, 9, 7)])
def test_conv_forward_ignores_fast_gain(case):
    """The reference's conv forward (concord/packed_b.py:2046-2065) runs on
    the ungated weight: fast_gain < 1 gates only the linear layer's forward
    (1762-1772).  On each conv path (implicit, 1 x 1 linear, im2col) a layer
    with fast_gain 0.25 gives the same output bits as one with 1.0."""
    import concord_amd as ca
    cin, cout, k, stride, pad, B, H, W = case
    torch.manual_seed(sum(case) + 3)
    W0 = torch.randn(cout, cin, k, k) * 0.05
    x = torch.randn(B, cin, H, W, device=DEV).to(torch.bfloat16)
    outs = []
    for fg in (1.0, 0.25):
        conv = ca.ConcordConv2dPackedB(cin, cout, k, stride=stride, padding=pad, bias=True, device=DEV)
        conv.load_weights(W0)
        conv.fast_gain = fg
        with torch.no_grad():
            outs.append(conv(x).float().cpu())
    sync()
    assert torch.equal(outs[0], outs[1])


# ---------------------------------------------------------------- implicit GEMM
# (cin, cout, k, stride, pad, B, H, W); channels multiples of 64, so these
# take the implicit-GEMM path: ragged spatial sizes (positions not a multiple
# of the 256-row tile), stride 2, mixed strides / paddings, a 5 x 5 kernel,
# an image row wider than a 64-position stage
IMPLICIT = [
    (64, 64, 3, 1, 1, 2, 20, 24),
    (128, 64, 3, 2, 1, 2, 17, 15),
    (64, 128, 3, 1, 1, 1, 9, 70),
    (64, 64, (3, 1), (2, 1), (1, 0), 3, 11, 13),
    (64, 192, 5, 1, 2, 1, 12, 10),
    (192, 64, 3, 2, 0, 2, 16, 16),
    # 49 taps: more than the gather's per-row tap masks hold (the general path)
    (64, 64, 7, 2, 3, 1, 13, 11),
]
# 320 channels: the WGRAD takes 128 x 256 tiles (the cases above 256 x 128)
WGRAD_128_ROWS = (320, 320, 3, 1, 1, 2, 24, 24)


def _geom(case):
    from torch.nn.modules.utils import _pair
    cin, cout, k, stride, pad, B, H, W = case
    (kh, kw), (sh, sw), (ph, pw) = _pair(k), _pair(stride), _pair(pad)
    return (B, cin, H, W, cout, kh, kw, sh, sw, ph, pw)


def test_conv_paths():
    """SDXL's convs take the expected path: the 4-channel latent input and
    output through the patch matrix, every resnet / downsample conv by
    implicit GEMM, 1 x 1 projections through the linear path."""
    import concord_amd as ca
    cases = [((4, 320, 3, 1, 1), (2, 4, 128, 128), 'im2col'),
             ((320, 320, 3, 1, 1), (2, 320, 128, 128), 'implicit'),
             ((320, 320, 3, 2, 1), (2, 320, 128, 128), 'implicit'),
             ((640, 1280, 3, 1, 1), (2, 640, 32, 32), 'implicit'),
             ((960, 640, 1, 1, 0), (2, 960, 64, 64), 'linear'),
             ((320, 4, 3, 1, 1), (2, 320, 128, 128), 'im2col')]
    for (cin, cout, k, s, p), shape, want in cases:
        conv = ca.ConcordConv2dPackedB(cin, cout, k, stride=s, padding=p, device=DEV)
        x = torch.empty(shape, device=DEV, dtype=torch.bfloat16)
        assert conv.conv_path(x) == want, ((cin, cout, k, s, p), shape)


@pytest.mark.parametrize("case", IMPLICIT + [WGRAD_128_ROWS])
def test_implicit_products_match_fp32(case):
    """y, dx, the weight gradient the update consumes and the bias gradient
    of the implicit-GEMM path against fp32 torch convolutions of the decoded
    weight (rel-L2 <= 1e-2)."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    cin, cout, k, stride, pad, B, H, W = case
    torch.manual_seed(7)
    conv = ca.ConcordConv2dPackedB(cin, cout, k, stride=stride, padding=pad, bias=True, device=DEV, lr=1e-3)
    with torch.no_grad():
        conv.bias.copy_((torch.randn(cout) * 0.1).to(torch.bfloat16))
    Wd = conv.weight.detach().float().clone()
    bd = conv.bias.detach().float().clone()
    x = torch.randn(B, cin, H, W, device=DEV).to(torch.bfloat16)
    assert conv.conv_path(x) == 'implicit'
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
    torch.backends.cudnn.allow_tf32 = False
    xf = x.float().requires_grad_(True)
    yf = F.conv2d(xf, Wd, bd, stride=stride, padding=pad)
    yf.backward(gy.float())
    gw = torch.nn.grad.conv2d_weight(x.float(), Wd.shape, gy.float(), stride=stride, padding=pad)
    assert y.shape == yf.shape and xc.grad.shape == x.shape
    assert rel_l2(host(y.float()), host(yf)) < 1e-2
    assert rel_l2(host(xc.grad.float()), host(xf.grad)) < 1e-2
    assert rel_l2(host(cap[0].float()), host(gw.reshape(cout, -1))) < 1e-2
    assert rel_l2(host(conv.bias.grad.float()), host(gy.float().sum(dim=(0, 2, 3)))) < 1e-2


@pytest.mark.parametrize("case", IMPLICIT[:3] + IMPLICIT[4:5] + IMPLICIT[-1:] + [WGRAD_128_ROWS])
def test_implicit_abi_products_float64(oracle, case):
    """The three C-ABI products on random bf16 operands against float64
    references: each output is one fp32 sum rounded once to bf16, so
    |got - exact| <= 2^-8 |exact| + 2^-17 sum |terms| elementwise."""
    from concord_amd import _lib as C
    from concord_amd import packed_b as pb
    geom = _geom(case)
    B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw = geom
    T = kh * kw
    Ho, Wo = (H + 2 * ph - kh) // sh + 1, (W + 2 * pw - kw) // sw + 1
    g = torch.Generator().manual_seed(11)
    x = torch.randn(B, H, W, Cin, generator=g).to(torch.bfloat16)
    dy = torch.randn(B, Ho, Wo, Cout, generator=g).to(torch.bfloat16)
    wt = (torch.randn(Cout, T, Cin, generator=g) * 0.1).to(torch.bfloat16)
    bias = (torch.randn(Cout, generator=g) * 0.1).to(torch.bfloat16)
    xd, dyd, wtd, bd = x.to(DEV), dy.to(DEV), wt.to(DEV), bias.to(DEV)
    ws = pb._conv_workspace(torch.device(DEV), geom)
    st = C.stream_of(torch.device(DEV))
    y = torch.empty(B, Ho, Wo, Cout, dtype=torch.bfloat16, device=DEV)
    dx = torch.empty(B, H, W, Cin, dtype=torch.bfloat16, device=DEV)
    gt = torch.empty(Cout, T, Cin, dtype=torch.bfloat16, device=DEV)
    C.check(C.lib().concord_conv_fwd(C.ptr(xd), C.ptr(wtd), C.ptr(bd), C.ptr(y), *geom, C.ptr(ws), ws.numel(), st),
            "conv_fwd")
    C.check(C.lib().concord_conv_dgrad(C.ptr(dyd), C.ptr(wtd), C.ptr(dx), *geom, C.ptr(ws), ws.numel(), st),
            "conv_dgrad")
    C.check(C.lib().concord_conv_wgrad(C.ptr(dyd), C.ptr(xd), C.ptr(gt), *geom, C.ptr(ws), ws.numel(), st),
            "conv_wgrad")
    sync()
    x64 = x.double().permute(0, 3, 1, 2)
    W64 = wt.double().view(Cout, kh, kw, Cin).permute(0, 3, 1, 2)
    dy64 = dy.double().permute(0, 3, 1, 2)
    checks = [
        (y, F.conv2d(x64, W64, bias.double(), stride=(sh, sw), padding=(ph, pw)).permute(0, 2, 3, 1),
         F.conv2d(x64.abs(), W64.abs(), bias.double().abs(), stride=(sh, sw), padding=(ph, pw)).permute(0, 2, 3, 1)),
        (dx, torch.nn.grad.conv2d_input(x64.shape, W64, dy64, stride=(sh, sw), padding=(ph, pw)).permute(0, 2, 3, 1),
         torch.nn.grad.conv2d_input(x64.shape, W64.abs(), dy64.abs(), stride=(sh, sw),
                                    padding=(ph, pw)).permute(0, 2, 3, 1)),
        (gt, torch.nn.grad.conv2d_weight(x64, W64.shape, dy64, stride=(sh, sw), padding=(ph, pw))
         .permute(0, 2, 3, 1).reshape(Cout, T, Cin),
         torch.nn.grad.conv2d_weight(x64.abs(), W64.shape, dy64.abs(), stride=(sh, sw), padding=(ph, pw))
         .permute(0, 2, 3, 1).reshape(Cout, T, Cin)),
    ]
    for got, exact, mag in checks:
        gv = oracle.bf16_bits_to_f32(host(got)).astype(np.float64)
        ex, mg = exact.numpy(), mag.numpy()
        tol = 2.0 ** -8 * np.abs(ex) + 2.0 ** -17 * mg
        assert np.all(np.abs(gv - ex) <= tol), float(np.max(np.abs(gv - ex) - tol))


@pytest.mark.parametrize("case", IMPLICIT)
def test_conv_wgrad_vhat_matches_separate_calls(oracle, case):
    """concord_conv_wgrad_vhat against concord_conv_wgrad +
    concord_conv_grad_from_taps + concord_vhat_ema on the same operands:
    gt, the packed-order gradient, v_row, v_col, sum_v_inv, the salt and the
    zeroed watermarks bit-identical (3 x 3 kernels take the fused reorder,
    the 3 x 1 and 5 x 5 cases the two-pass one); the bias gradient within fp32
    summation error of the float64 sum of dy, rounded once to bf16."""
    from concord_amd import _lib as C
    from concord_amd import packed_b as pb
    geom = _geom(case)
    B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw = geom
    T = kh * kw
    Ho, Wo = (H + 2 * ph - kh) // sh + 1, (W + 2 * pw - kw) // sw + 1
    M, K = B * Ho * Wo, Cin * T
    g = torch.Generator().manual_seed(13)
    x = torch.randn(B, H, W, Cin, generator=g).to(torch.bfloat16).to(DEV)
    dy = (torch.randn(B, Ho, Wo, Cout, generator=g) * 0.1).to(torch.bfloat16).to(DEV)
    vr0 = torch.rand(Cout, generator=g).to(DEV)
    vc0 = torch.rand(K, generator=g).to(DEV)
    dev = torch.device(DEV)
    st = C.stream_of(dev)
    gws = pb._conv_workspace(dev, geom)
    outs = []
    for fused in (False, True):
        gt = torch.empty(Cout, K, dtype=torch.bfloat16, device=DEV)
        gw = torch.empty(Cout, K, dtype=torch.bfloat16, device=DEV)
        vr, vc = vr0.clone(), vc0.clone()
        svi = torch.zeros(1, device=DEV)
        rm = torch.full((Cout,), 5, dtype=torch.int32, device=DEV)
        cm = torch.full((K,), 5, dtype=torch.int32, device=DEV)
        salt = torch.full((1,), 40, dtype=torch.int32, device=DEV)
        gb = torch.empty(Cout, dtype=torch.bfloat16, device=DEV)
        if fused:
            ws = pb._workspace(dev, Cout, K, M)
            C.check(C.lib().concord_conv_wgrad_vhat(
                C.ptr(dy), C.ptr(x), C.ptr(gt), C.ptr(gw), gw.stride(0), *geom, 0.999, C.ptr(vr), C.ptr(vc),
                C.ptr(svi), C.ptr(rm), C.ptr(cm), C.ptr(salt), C.ptr(gb), C.ptr(ws), ws.numel(), C.ptr(gws),
                gws.numel(), st), "conv_wgrad_vhat")
        else:
            C.check(C.lib().concord_conv_wgrad(C.ptr(dy), C.ptr(x), C.ptr(gt), *geom, C.ptr(gws), gws.numel(), st),
                    "conv_wgrad")
            C.check(C.lib().concord_conv_grad_from_taps(C.ptr(gt), Cout, Cin, T, C.ptr(gw), gw.stride(0), st),
                    "conv_grad_from_taps")
            pb.vhat_ema(gw, vr, vc, svi, 0.999, rm, cm, salt)
        sync()
        outs.append([host(t).copy() for t in (gt, gw, vr, vc, svi, rm, cm, salt)] + [host(gb).copy()])
    for a, b in zip(outs[0][:8], outs[1][:8]):
        np.testing.assert_array_equal(a, b)
    assert int(outs[1][7][0]) == 41 and not outs[1][5].any() and not outs[1][6].any()
    d64 = oracle.bf16_bits_to_f32(host(dy)).astype(np.float64)
    exact = d64.reshape(M, Cout).sum(axis=0)
    mag = np.abs(d64.reshape(M, Cout)).sum(axis=0)
    got = oracle.bf16_bits_to_f32(outs[1][8]).astype(np.float64)
    assert np.all(np.abs(got - exact) <= 2.0 ** -8 * np.abs(exact) + 2.0 ** -11 * mag)


@pytest.mark.parametrize("gain", [1.0, 0.37])
def test_weight_taps_bit_exact(oracle, gain):
    """W'[n][t][c] is the oracle's (gated) decode of word (n, c * taps + t)."""
    from concord_amd import _lib as C
    from gpu_util import dev, rand_state
    rng = np.random.default_rng(5)
    for Cout, Cin, T in [(64, 64, 9), (37, 130, 9), (5, 7, 25), (3, 64, 1)]:
        packed, re, ce = rand_state(rng, Cout, Cin * T, sf=(-32768, 32768), exp=(-8, 7), col=(-8, 7))
        wt = torch.empty(Cout, T, Cin, dtype=torch.bfloat16, device=DEV)
        # the device copies stay referenced until the kernel has run
        pd, red, ced = dev(packed), dev(re), dev(ce)
        C.check(C.lib().concord_conv_weight_taps(C.ptr(pd), Cin * T, C.ptr(red), C.ptr(ced), Cout, Cin, T, 15, gain,
                                                 C.ptr(wt), C.stream_of(torch.device(DEV))), "conv_weight_taps")
        sync()
        want = (oracle.materialize(packed, re, ce) if gain == 1.0 else
                oracle.materialize_gated(packed, re, ce, gain))
        np.testing.assert_array_equal(host(wt), want.reshape(Cout, Cin, T).transpose(0, 2, 1))


def test_grad_from_taps_is_the_permutation():
    from concord_amd import _lib as C
    for Cout, Cin, T in [(64, 64, 9), (37, 130, 9), (5, 7, 25), (3, 64, 1)]:
        gt = torch.randint(-2 ** 15, 2 ** 15, (Cout, T, Cin), dtype=torch.int16, device=DEV).view(torch.bfloat16)
        g = torch.full((Cout, Cin * T + 3), 7, dtype=torch.int16, device=DEV).view(torch.bfloat16)
        C.check(C.lib().concord_conv_grad_from_taps(C.ptr(gt), Cout, Cin, T, C.ptr(g), g.stride(0),
                                                    C.stream_of(torch.device(DEV))), "conv_grad_from_taps")
        sync()
        want = host(gt).transpose(0, 2, 1).reshape(Cout, Cin * T)
        np.testing.assert_array_equal(host(g)[:, :Cin * T], want)
        assert (host(g)[:, Cin * T:] == 7).all()


@pytest.mark.parametrize("case", [IMPLICIT[0], IMPLICIT[1]])
def test_implicit_layer_state_vs_oracle(oracle, case):
    """Three training steps of an implicit-GEMM conv layer (default flags,
    coh_pre on): the v-hat, packed words, exponents after rebalance and the
    bf16 forward weight, bit-exact against the oracle fed each step's
    captured bf16 gradient (in the packed (c, tap) order)."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    O = oracle
    cin, cout, k, stride, pad, B, H, W = case
    torch.manual_seed(21)
    conv = ca.ConcordConv2dPackedB(cin, cout, k, stride=stride, padding=pad, bias=True, device=DEV, lr=2e-3)
    W0 = torch.randn(cout, cin * k * k) * 0.05
    conv.load_weights(W0)
    p0, r0, c0 = O.load_weights(W0.numpy())
    np.testing.assert_array_equal(host(conv.packed_w), p0)
    K = cin * k * k
    st = [p0.copy(), r0.copy(), c0.copy(), np.zeros(cout, np.float32), np.zeros(K, np.float32)]
    coh = np.ones((cout, K), np.float32)
    flags = O.MASS_PRESERVE | O.APPLY_CHASE | O.TRACK_REBALANCE | O.GF_TRUST_REGION | O.FIXED_COH | O.COHPRE
    P = O.UpdateParams(alpha=0.1, beta1=0.0, weight_decay=0.0, step_cap=10.0, v_scale=0.0, precond_p=0.5,
                       gf_consol=0.0, drift_cancel_C=conv.drift_cancel_C, alpha_v_fast=0.001, wd_sv=0.0,
                       wd_sf=0.0, gf_trust_delta_sq=1.0, gate_gain=1.0, mantissa_bias=15)
    for step in range(3):
        salt_next = int(host(pb._get_step_counter(DEV))[0]) + 1
        x = torch.randn(B, cin, H, W, device=DEV).to(torch.bfloat16).requires_grad_(True)
        cap = []
        pb._DEBUG_CAPTURE = cap
        try:
            y = conv(x)
            y.backward((torch.randn_like(y.float()) * 3e-2).to(torch.bfloat16))
        finally:
            pb._DEBUG_CAPTURE = None
        conv.rebalance()
        sync()
        g = host(cap[0])
        svi = O.vhat_ema(g, st[3], st[4], 0.999)
        rm = np.zeros(cout, np.int32)
        cm = np.zeros(K, np.int32)
        S = O.UpdateScalars(lr=2e-3, eps=1e-10, chase_floor=0.9, leak_floor=0.999, v_bc=1.0, salt=salt_next,
                            consolidate=1)
        O.apply_adamw(st[0], g, None, st[1], st[2], rm, cm, st[3], st[4], svi, coh, P, S, flags)
        O.rebalance(st[0], st[1], st[2], rm, cm, seed=step + 1)
        np.testing.assert_array_equal(host(conv.v_row), st[3])
        np.testing.assert_array_equal(host(conv.v_col), st[4])
        np.testing.assert_array_equal(host(conv.packed_w), st[0])
        np.testing.assert_array_equal(host(conv.row_exp), st[1])
        np.testing.assert_array_equal(host(conv.col_exp), st[2])
    np.testing.assert_array_equal(host(conv.get_weight()), O.materialize(st[0], st[1], st[2]))


@pytest.mark.parametrize("case", [(640, 640, 3, 1, 1, 2, 64, 64), (320, 320, 3, 1, 1, 2, 128, 128)])
def test_sdxl_conv_layer_state_vs_oracle(oracle, case):
    """One training step of an SDXL-sized 3 x 3 conv layer (640 channels at
    64^2 and 320 at 128^2, batch 2): the WGRAD takes the 128 x 256 tiles and
    a split reduction with the v-hat partials (concord_conv_wgrad_vhat).
    v-hat, packed words and exponents after the rebalance bit-exact against
    the oracle fed the captured bf16 gradient, as the toy geometries above."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    O = oracle
    cin, cout, k, stride, pad, B, H, W = case
    torch.manual_seed(23)
    conv = ca.ConcordConv2dPackedB(cin, cout, k, stride=stride, padding=pad, bias=True, device=DEV, lr=5e-4)
    W0 = torch.randn(cout, cin * k * k) * 0.02
    conv.load_weights(W0)
    p0, r0, c0 = O.load_weights(W0.numpy())
    K = cin * k * k
    st = [p0.copy(), r0.copy(), c0.copy(), np.zeros(cout, np.float32), np.zeros(K, np.float32)]
    coh = np.ones((cout, K), np.float32)
    flags = O.MASS_PRESERVE | O.APPLY_CHASE | O.TRACK_REBALANCE | O.GF_TRUST_REGION | O.FIXED_COH | O.COHPRE
    P = O.UpdateParams(alpha=0.1, beta1=0.0, weight_decay=0.0, step_cap=10.0, v_scale=0.0, precond_p=0.5,
                       gf_consol=0.0, drift_cancel_C=conv.drift_cancel_C, alpha_v_fast=0.001, wd_sv=0.0,
                       wd_sf=0.0, gf_trust_delta_sq=1.0, gate_gain=1.0, mantissa_bias=15)
    salt_next = int(host(pb._get_step_counter(DEV))[0]) + 1
    x = torch.randn(B, cin, H, W, device=DEV).to(torch.bfloat16).requires_grad_(True)
    assert conv.conv_path(x) == 'implicit'
    cap = []
    pb._DEBUG_CAPTURE = cap
    try:
        y = conv(x)
        y.backward((torch.randn_like(y.float()) * 1e-3).to(torch.bfloat16))
    finally:
        pb._DEBUG_CAPTURE = None
    conv.rebalance()
    sync()
    g = host(cap[0])
    svi = O.vhat_ema(g, st[3], st[4], 0.999)
    rm = np.zeros(cout, np.int32)
    cm = np.zeros(K, np.int32)
    S = O.UpdateScalars(lr=5e-4, eps=1e-10, chase_floor=0.9, leak_floor=0.999, v_bc=1.0, salt=salt_next,
                        consolidate=1)
    O.apply_adamw(st[0], g, None, st[1], st[2], rm, cm, st[3], st[4], svi, coh, P, S, flags)
    O.rebalance(st[0], st[1], st[2], rm, cm, seed=1)
    np.testing.assert_array_equal(host(conv.v_row), st[3])
    np.testing.assert_array_equal(host(conv.v_col), st[4])
    np.testing.assert_array_equal(host(conv.packed_w), st[0])
    np.testing.assert_array_equal(host(conv.row_exp), st[1])
    np.testing.assert_array_equal(host(conv.col_exp), st[2])
    assert (st[0] != p0).any()


# SDXL-UNet conv shapes at batch 2 of a 1024 px latent: the 3 x 3 resnet
# convs per level (320 ch at 128^2, 640 at 64^2, 1280 at 32^2), a stride-2
# downsample, and the level-crossing 640 -> 1280 conv
SDXL_CONV = [(320, 320, 3, 1, 1, 2, 128, 128), (640, 640, 3, 1, 1, 2, 64, 64), (1280, 1280, 3, 1, 1, 2, 32, 32),
             (640, 640, 3, 2, 1, 2, 64, 64), (640, 1280, 3, 1, 1, 2, 32, 32)]


@pytest.mark.parametrize("case", SDXL_CONV)
def test_sdxl_conv_shapes(case):
    """One training step of each SDXL conv shape on the implicit path: y, dx
    and the captured weight gradient against fp32 torch convolutions of the
    decoded weight (rel-L2 <= 1e-2), finite packed state after the update."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    cin, cout, k, stride, pad, B, H, W = case
    torch.manual_seed(3)
    conv = ca.ConcordConv2dPackedB(cin, cout, k, stride=stride, padding=pad, bias=True, device=DEV, lr=5e-4)
    Wd = conv.weight.detach().float().clone()
    x = torch.randn(B, cin, H, W, device=DEV).to(torch.bfloat16)
    assert conv.conv_path(x) == 'implicit'
    xc = x.clone().requires_grad_(True)
    cap = []
    pb._DEBUG_CAPTURE = cap
    try:
        y = conv(xc)
        gy = (torch.randn_like(y.float()) * 1e-3).to(torch.bfloat16)
        y.backward(gy)
    finally:
        pb._DEBUG_CAPTURE = None
    conv.rebalance()
    sync()
    torch.backends.cudnn.allow_tf32 = False
    xf = x.float().requires_grad_(True)
    yf = F.conv2d(xf, Wd, conv.bias.detach().float(), stride=stride, padding=pad)
    yf.backward(gy.float())
    gw = torch.nn.grad.conv2d_weight(x.float(), Wd.shape, gy.float(), stride=stride, padding=pad)
    assert rel_l2(host(y.float()), host(yf)) < 1e-2
    assert rel_l2(host(xc.grad.float()), host(xf.grad)) < 1e-2
    assert rel_l2(host(cap[0].float()), host(gw.reshape(cout, -1))) < 1e-2
    assert torch.isfinite(conv.get_weight().float()).all().item()
