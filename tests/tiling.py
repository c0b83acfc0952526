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
