"""The FC transport operator the swap router propagates omission errors with.

The spectral corrector of the previous layer publishes, per anchor pair, a
phase ``theta`` and an affinity ``g`` per overlap window and frequency
(P/matrix_world_spectral_residual.py:597-658).  Transporting a map on the
attention block grid by a fraction ``a`` of that phase means: lift the map to
the corrector's output grid (bilinear), cut it into the corrector's windows
(reflect padding, square-root Hann weights, optional 2x average pooling to the
transport grid), multiply each window's spectrum by exp(i a g theta), return
to pixels, overlap-add with the same weights, and average back onto the block
grid.  The operator is the identity plus the change this makes relative to the
zero-phase round trip, so a = 0 (or theta = 0) gives exactly the identity
(``_transport_matrix``, P/fc_pasm_swap_routing.py:116-269).

``fc_transport_operator`` builds it as an [S, S] matrix (output x input) on the
transport tensors' device by transporting the S unit maps at once, with torch
(FFT, unfold/fold); the router calls it for each skipped frame of a pair.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn.functional as F


def _window(h: int, w: int, device) -> torch.Tensor:
    wy = torch.hann_window(h, periodic=False, device=device, dtype=torch.float32)
    wx = torch.hann_window(w, periodic=False, device=device, dtype=torch.float32)
    return (wy[:, None] * wx[None, :]).clamp_min(0.0).sqrt()


def transport_maps(transport: dict, pair, maps: torch.Tensor, exponent: float) -> torch.Tensor:
    """Change of ``maps`` [N, C, h, w] (the attention block grid) under the pair's
    transport at ``exponent``: transported minus zero-phase round trip."""
    entry = transport["pairs"][pair]
    dev = maps.device
    theta = entry["theta"].to(device=dev, dtype=torch.float32)
    gain = entry["affinity"].to(device=dev, dtype=torch.float32)
    oh, ow = (int(v) for v in transport["output_shape"])
    th, tw = (int(v) for v in transport["transport_shape"])
    wh, ww = (int(v) for v in transport["window_shape"])
    sh, sw = (int(v) for v in transport["stride"])
    ph, pw = (int(v) for v in transport["padding"])
    gh, gw = (int(v) for v in transport["tile_grid"])
    tiles_n = gh * gw
    if theta.shape[0] != tiles_n or gain.shape != theta.shape:
        raise RuntimeError("FC transport tiles do not match the overlap grid")
    n, c, h, w = maps.shape
    win = _window(wh, ww, dev)
    up = F.interpolate(maps.float(), size=(oh, ow), mode="bilinear", align_corners=False)
    padded = F.pad(up, (pw, pw, ph, ph), mode="reflect")
    cols = F.unfold(padded, kernel_size=(wh, ww), stride=(sh, sw))      # [n, c*wh*ww, tiles]
    if cols.shape[-1] != tiles_n:
        raise RuntimeError("FC transport windows do not match the tile grid")
    tiles = cols.reshape(n, c, wh, ww, tiles_n).permute(0, 4, 1, 2, 3) * win
    pooled = (th, tw) != (wh, ww)
    if pooled:
        tiles = F.avg_pool2d(tiles.reshape(n * tiles_n, c, wh, ww), kernel_size=2, stride=2,
                             ceil_mode=True, count_include_pad=False).reshape(n, tiles_n, c, th, tw)
    spec = torch.fft.rfft2(tiles, dim=(-2, -1))
    if theta.shape[-2:] != spec.shape[-2:]:
        raise RuntimeError("FC transport spectrum has an invalid shape")
    rot = torch.polar(torch.ones_like(theta), float(exponent) * gain * theta)
    moved = torch.fft.irfft2(spec * rot[None, :, None], s=(th, tw), dim=(-2, -1))
    still = torch.fft.irfft2(spec, s=(th, tw), dim=(-2, -1))
    if pooled:
        moved, still = (F.interpolate(x.reshape(n * tiles_n, c, th, tw), size=(wh, ww),
                                      mode="bilinear", align_corners=False)
                        .reshape(n, tiles_n, c, wh, ww) for x in (moved, still))
    full_h, full_w = oh + 2 * ph, ow + 2 * pw
    norm = F.fold((win * win).reshape(1, wh * ww, 1).expand(1, wh * ww, tiles_n),
                  output_size=(full_h, full_w), kernel_size=(wh, ww), stride=(sh, sw))
    norm = norm[:, :, ph:ph + oh, pw:pw + ow].clamp_min(1e-8)

    def overlap_add(x):
        cols_ = (x * win).permute(0, 2, 3, 4, 1).reshape(n, c * wh * ww, tiles_n)
        out = F.fold(cols_, output_size=(full_h, full_w), kernel_size=(wh, ww), stride=(sh, sw))
        return out[:, :, ph:ph + oh, pw:pw + ow] / norm

    diff = overlap_add(moved) - overlap_add(still)
    bh, bw = math.ceil(oh / h), math.ceil(ow / w)
    delta = F.avg_pool2d(diff, kernel_size=(bh, bw), stride=(bh, bw), ceil_mode=True,
                         count_include_pad=False)
    if tuple(delta.shape[-2:]) != (h, w):
        raise RuntimeError("FC transport did not return the attention grid")
    return delta


def fc_transport_operator(transport: Optional[dict], pair, spatial_shape,
                          exponent: float) -> Optional[torch.Tensor]:
    """The pair's transport operator on the ``spatial_shape`` block grid at
    ``exponent`` ([S, S], output x input), or None when the transport holds no
    usable entry for the pair (the router then uses the identity).  Cached in
    the pair's entry per (grid, exponent, device)."""
    if not isinstance(transport, dict):
        return None
    entry = transport.get("pairs", {}).get(pair)
    if not isinstance(entry, dict):
        return None
    theta, gain = entry.get("theta"), entry.get("affinity")
    if (not isinstance(theta, torch.Tensor) or not isinstance(gain, torch.Tensor)
            or theta.ndim != 3 or gain.shape != theta.shape):
        return None
    h, w = (int(v) for v in spatial_shape)
    cache = entry.setdefault("_attention_operator_cache", {})
    key = (h, w, round(float(exponent), 12), str(theta.device))
    if key in cache:
        return cache[key]
    s = h * w
    eye = torch.eye(s, device=theta.device, dtype=torch.float32)
    delta = transport_maps(transport, pair, eye.reshape(s, 1, h, w), exponent)
    # row j of the stacked changes is the change of unit map j: transpose to output x input
    op = (eye + delta.reshape(s, s)).transpose(0, 1).contiguous()
    cache[key] = op
    return op
