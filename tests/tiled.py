"""numpy packers for the tiled cache layouts (test infrastructure).

An independent statement of the layouts the library's producers write
(csrc/kvlayout.h), used to build tiled caches from plain arrays on the host
and to check the device producers byte for byte. Vectorised index arithmetic,
not a port of the device code.
"""
from __future__ import annotations

import numpy as np


def _lanes():
    l = np.arange(64)
    return l, l & 15, l >> 4  # lane, col, grp


def t16_index(hd: int):
    """(key, dim) of each half in one block's K area and V area, as arrays of
    shape [32*hd] each: K area element e holds K[key_k[e], dim_k[e]], V area
    element e holds V[dim_v[e]][key_v[e]]."""
    ns, nt = hd // 32, hd // 16
    l, col, grp = _lanes()
    j = np.arange(8)
    T, s = np.meshgrid(np.arange(2), np.arange(ns), indexing="ij")
    # order: ((T*ns + s)*64 + l)*8 + j
    key_k = (8 * (col // 4) + (col % 4))[None, None, :, None] + 4 * T[:, :, None, None] + 0 * j
    dim_k = 32 * s[:, :, None, None] + 8 * grp[None, None, :, None] + j[None, None, None, :]
    key_k = np.broadcast_to(key_k, (2, ns, 64, 8)).ravel()
    dim_k = np.broadcast_to(dim_k, (2, ns, 64, 8)).ravel()
    t = np.arange(nt)
    # order: (t*64 + l)*8 + j
    dim_v = (16 * t[:, None, None] + col[None, :, None]) + 0 * j[None, None, :]
    key_v = (8 * grp[None, :, None] + j[None, None, :]) + 0 * t[:, None, None]
    return key_k, dim_k, np.broadcast_to(key_v, (nt, 64, 8)).ravel(), np.broadcast_to(dim_v, (nt, 64, 8)).ravel()


def pack_t16(k, v, kv: int, hd: int, cap: int, live: int | None = None) -> np.ndarray:
    """Reference-layout f16 bits K [kv][cap][hd], V [kv][hd][cap] -> tiled
    uint16 [kv][nblk][2][32*hd]; positions >= live (default cap) are zero."""
    live = cap if live is None else live
    nblk = (cap + 31) // 32
    k = np.asarray(k, np.uint16).reshape(kv, cap, hd)
    v = np.asarray(v, np.uint16).reshape(kv, hd, cap)
    kk = np.zeros((kv, nblk * 32, hd), np.uint16)
    vv = np.zeros((kv, hd, nblk * 32), np.uint16)
    kk[:, :live] = k[:, :live]
    vv[:, :, :live] = v[:, :, :live]
    key_k, dim_k, key_v, dim_v = t16_index(hd)
    out = np.zeros((kv, nblk, 2, 32 * hd), np.uint16)
    for b in range(nblk):
        out[:, b, 0] = kk[:, 32 * b + key_k, dim_k]
        out[:, b, 1] = vv[:, dim_v, 32 * b + key_v]
    return out.ravel()


def unpack_t16(data, kv: int, hd: int, cap: int):
    """Inverse of pack_t16: tiled uint16 -> (K [kv][cap][hd], V [kv][hd][cap])."""
    nblk = (cap + 31) // 32
    d = np.asarray(data, np.uint16).reshape(kv, nblk, 2, 32 * hd)
    key_k, dim_k, key_v, dim_v = t16_index(hd)
    kk = np.zeros((kv, nblk * 32, hd), np.uint16)
    vv = np.zeros((kv, hd, nblk * 32), np.uint16)
    for b in range(nblk):
        kk[:, 32 * b + key_k, dim_k] = d[:, b, 0]
        vv[:, dim_v, 32 * b + key_v] = d[:, b, 1]
    return np.ascontiguousarray(kk[:, :cap]), np.ascontiguousarray(vv[:, :, :cap])


def q8_block_bytes(hd: int) -> int:
    return 2 * 32 * hd + 2 * 32 * (hd // 32) * 2


def q8_index(hd: int):
    """(key, dim) of each byte of a block's K-code and V-code areas."""
    ns, nt = hd // 32, hd // 16
    l, col, grp = _lanes()
    e = np.arange(16)
    # K: ((T*(ns/2) + sp)*64 + l)*16 + e, s = 2sp + e//8, j = e%8
    T, sp = np.meshgrid(np.arange(2), np.arange(ns // 2), indexing="ij")
    s = 2 * sp[:, :, None, None] + (e // 8)[None, None, None, :]
    key_k = (8 * (col // 4) + (col % 4))[None, None, :, None] + 4 * T[:, :, None, None]
    dim_k = 32 * s + 8 * grp[None, None, :, None] + (e % 8)[None, None, None, :]
    key_k = np.broadcast_to(key_k, (2, ns // 2, 64, 16)).ravel()
    dim_k = np.broadcast_to(dim_k, (2, ns // 2, 64, 16)).ravel()
    # V: ((t//2)*64 + l)*16 + 8*(t%2) + j
    tp = np.arange(nt // 2)
    t = 2 * tp[:, None, None] + (e // 8)[None, None, :]
    dim_v = 16 * t + col[None, :, None]
    key_v = 8 * grp[None, :, None] + (e % 8)[None, None, :] + 0 * tp[:, None, None]
    return key_k, dim_k, np.broadcast_to(key_v, (nt // 2, 64, 16)).ravel(), np.broadcast_to(dim_v, (nt // 2, 64, 16)).ravel()


def pack_q8(kc, ks, vc, vs, slots: int, kv: int, hd: int, cap: int) -> np.ndarray:
    """Plain Q8_0 arrays -> the tiled cache bytes (int8).
    kc [slots][kv][cap][hd] int8, vc [slots][kv][hd][cap] int8,
    ks, vs [slots][kv][cap][hd/32] f16 bits."""
    nb = hd // 32
    nblk = (cap + 31) // 32
    kc = np.asarray(kc, np.int8).reshape(slots * kv, cap, hd)
    vc = np.asarray(vc, np.int8).reshape(slots * kv, hd, cap)
    ks = np.asarray(ks, np.uint16).reshape(slots * kv, cap, nb)
    vs = np.asarray(vs, np.uint16).reshape(slots * kv, cap, nb)
    pad = nblk * 32 - cap
    if pad:
        kc = np.pad(kc, ((0, 0), (0, pad), (0, 0)))
        vc = np.pad(vc, ((0, 0), (0, 0), (0, pad)))
        ks = np.pad(ks, ((0, 0), (0, pad), (0, 0)))
        vs = np.pad(vs, ((0, 0), (0, pad), (0, 0)))
    key_k, dim_k, key_v, dim_v = q8_index(hd)
    bb = q8_block_bytes(hd)
    out = np.zeros((slots * kv, nblk, bb), np.uint8)
    for b in range(nblk):
        # codes offset-binary: the sign bit flipped
        out[:, b, :32 * hd] = kc[:, 32 * b + key_k, dim_k].view(np.uint8) ^ 0x80
        out[:, b, 32 * hd:64 * hd] = vc[:, dim_v, 32 * b + key_v].view(np.uint8) ^ 0x80
        # scales dim-block-major: [nb][32 keys]
        out[:, b, 64 * hd:64 * hd + 64 * nb] = np.ascontiguousarray(
            ks[:, 32 * b:32 * b + 32].transpose(0, 2, 1)).reshape(-1, 32 * nb).view(np.uint8)
        out[:, b, 64 * hd + 64 * nb:] = np.ascontiguousarray(
            vs[:, 32 * b:32 * b + 32].transpose(0, 2, 1)).reshape(-1, 32 * nb).view(np.uint8)
    return out.ravel().view(np.int8)
