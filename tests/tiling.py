"""numpy statement of the tiled int8 weight layout the library's W8A8 and
W8A32 entry points take (include/nemotron_hip.h, Conventions): used by the
tests to lay out row-major weights, independently of the library's own
nh_tile_weights_i8 / nh_tile_weights_i8_host, which the tests check against
it.  A layout that disagreed with the kernels' MFMA operand order could not
reproduce the oracle's row-major results, which every GEMV/GEMM test checks."""
import numpy as np


def tile_16x64(w):
    """int8 [N][K] row-major -> the tiled byte stream: tile (nt, kt) of 1024
    bytes at (nt * KT + kt) * 1024, byte 16 * (16 g + r) + b holding
    W[16 nt + r][64 kt + 16 g + b], zero padded to N % 16 == 0, K % 64 == 0."""
    w = np.asarray(w, dtype=np.int8)
    n, k = w.shape
    np_, kp = -(-n // 16) * 16, -(-k // 64) * 64
    p = np.zeros((np_, kp), dtype=np.int8)
    p[:n, :k] = w
    t = p.reshape(np_ // 16, 16, kp // 64, 4, 16).transpose(0, 2, 3, 1, 4)  # [nt][kt][g][r][b]
    return np.ascontiguousarray(t).reshape(-1)


def tile_experts(w):
    """[E][N][K] -> E tiled matrices back to back."""
    return np.concatenate([tile_16x64(we) for we in w])


def tiled_bytes(n, k):
    return -(-n // 16) * 16 * -(-k // 64) * 64


def tile_int4(packed, k, n, zp):
    """The reference's packed [k][n] INT4 codes (low nibble first) -> the
    tiled INT4 layout: 512-byte tiles of 16 rows (n) x 64 codes (k); lane
    l = 16 g + r holds bytes [8 l, 8 l + 8), byte j = codes k = 64 kt + 16 g
    + 2 j (low nibble) and + 2 j + 1 (high); the zero point outside."""
    packed = np.asarray(packed, dtype=np.uint8)
    flat = np.empty(packed.size * 2, dtype=np.uint8)
    flat[0::2], flat[1::2] = packed & 15, packed >> 4
    codes = flat[:k * n].reshape(k, n).T  # [n][k]
    nt, kt = (n + 15) // 16, (k + 63) // 64
    full = np.full((nt * 16, kt * 64), zp, dtype=np.uint8)
    full[:n, :k] = codes
    t = full.reshape(nt, 16, kt, 4, 16).transpose(0, 2, 3, 1, 4)  # [nt][kt][g][r][16 codes]
    t = t.reshape(nt, kt, 64, 8, 2)
    return (t[..., 0] | (t[..., 1] << 4)).astype(np.uint8).ravel()
