"""CPU oracle for the Winograd F(2x2,3x3) gradients -- test infrastructure only.

Plain numpy float64 restatements of the two backward passes the device runs
through Winograd for 3x3 stride-1 dilation-1 layers.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may use this module,
and only as the checker.

The transform matrices are the ones the reference's forward shaders use
(conv2d_winograd_weights.comp:17-28 for G, conv2d_winograd_input.comp:24-37 for
B^T, conv2d_winograd_gemm_output.comp:46-63 for A^T); the reference has no
Winograd backward, so its parity target for these gradients is its CPU
implementation (torch's convolution_backward), which the tests compare with:

  dinput_via_forward   dx as the Winograd forward convolution of dy with the
                       flipped, channel-swapped filter at padding 2 - p
                       (oracle.conv2d_forward(..., winograd=True) does the
                       transform arithmetic in C).
  dweight_adjoint      dw = G^T (sum over tiles of (A dY A^T) * (B^T d B)) G,
                       the adjoint of the forward transform.

What pins them (tests/test_oracle_conv.py): CPU torch float64 dx / dw of the
golden Winograd fixtures to 1e-9 relative; brute force on a tiny case; planted
mistakes (unflipped filter, a wrong sign in A, a transposed G) that must fail.
"""
from __future__ import annotations

import numpy as np

# F(2x2,3x3) transforms (forward: U = G g G^T, V = B^T d B, Y = A^T M A).
G = np.array([[1.0, 0.0, 0.0], [0.5, 0.5, 0.5], [0.5, -0.5, 0.5], [0.0, 0.0, 1.0]])
BT = np.array([[1.0, 0.0, -1.0, 0.0], [0.0, 1.0, 1.0, 0.0], [0.0, -1.0, 1.0, 0.0], [0.0, 1.0, 0.0, -1.0]])
AT = np.array([[1.0, 1.0, 1.0, 0.0], [0.0, 1.0, -1.0, -1.0]])


def flipped_filter(w, groups):
    """Filter of a 3x3 layer's input gradient seen as a convolution:
    [G*C][O][3][3] from the layer's [G*O][C][3][3], taps reversed."""
    go, c, kh, kw = w.shape
    o = go // groups
    wt = w.reshape(groups, o, c, kh, kw).transpose(0, 2, 1, 3, 4)[..., ::-1, ::-1]
    return np.ascontiguousarray(wt.reshape(groups * c, o, kh, kw))


def dweight_adjoint(x, dy, padding=(1, 1), groups=1, at=AT, g=G):
    """Weight gradient [G*O][C][3][3] of the 3x3 stride-1 layer with input x
    [N][G*C][H][W] and output gradient dy [N][G*O][OH][OW], through the
    adjoint of the Winograd forward on 2x2 output tiles (4x4 input patches at
    stride 2 from (2 ty - ph, 2 tx - pw), zero outside the image; dy zero past
    its edge).  `at` and `g` are parameters only so tests can plant mistakes."""
    x = np.asarray(x, np.float64)
    dy = np.asarray(dy, np.float64)
    n, cin, h, w = x.shape
    _, cout, oh, ow = dy.shape
    ph, pw = padding
    c, o = cin // groups, cout // groups
    th, tw = (oh + 1) // 2, (ow + 1) // 2
    # zero-padded views covering every patch and tile
    xp = np.zeros((n, cin, 2 * th + 2, 2 * tw + 2))
    ys, xs = max(0, -ph), max(0, -pw)
    y0, x0 = max(0, ph), max(0, pw)
    hh = min(h, 2 * th + 2 - y0)
    ww = min(w, 2 * tw + 2 - x0)
    xp[:, :, y0:y0 + hh - ys, x0:x0 + ww - xs] = x[:, :, ys:hh, xs:ww]
    dyp = np.zeros((n, cout, 2 * th, 2 * tw))
    dyp[:, :, :oh, :ow] = dy
    bt = BT
    du = np.zeros((groups, o, c, 4, 4))
    for ty in range(th):
        for tx in range(tw):
            d = xp[:, :, 2 * ty:2 * ty + 4, 2 * tx:2 * tx + 4]          # [n][cin][4][4]
            v = np.einsum("ij,ncjk,lk->ncil", bt, d, bt)                # B^T d B
            gy = dyp[:, :, 2 * ty:2 * ty + 2, 2 * tx:2 * tx + 2]        # [n][cout][2][2]
            m = np.einsum("ij,noik,kl->nojl", at, gy, at)               # A dY A^T
            v = v.reshape(n, groups, c, 4, 4)
            m = m.reshape(n, groups, o, 4, 4)
            du += np.einsum("ngoij,ngcij->gocij", m, v)
    dw = np.einsum("ai,gocij,jb->gocab", g.T, du, g)                    # G^T dU G
    return dw.reshape(cout, c, 3, 3)
