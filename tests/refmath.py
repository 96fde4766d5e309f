"""Independent float64 formulations used to pin the oracle (test infrastructure).

Nothing here restates the oracle's code: NVFP4 weights are decoded to dense float64 matrices with
the OCP Microscaling spec's e2m1 value set and torch's float8_e4m3fn decoder, and the products are
plain numpy matmuls, so an index, nibble-order or scale mistake in the oracle shows up as a mismatch.
"""
import numpy as np

# OCP MX v1.0 FP4 (E2M1) values for codes 0..7; code | 8 is the negative.
E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float64)


def e2m1_decode(codes):
    codes = np.asarray(codes, dtype=np.int64)
    mag = E2M1_VALUES[codes & 7]
    return np.where(codes & 8, -mag, mag)


def e4m3_decode(bytes_):
    """unsigned e4m3 via torch.float8_e4m3fn (sign bit cleared); code 0x7F (NaN in e4m3fn) is
    decoded as the reference does, (1 + 7/8) * 2^8 = 480."""
    import torch
    b = np.asarray(bytes_, dtype=np.uint8) & 0x7F
    t = torch.from_numpy(b.copy()).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    return np.where(b == 0x7F, 480.0, t)


def blob_dense(blob, D, F):
    """Decode a reference-layout NVFP4 expert blob into dense float64 (gate [F,D], up [F,D],
    down [D,F]) including the per-tensor scales."""
    blob = np.asarray(blob, dtype=np.uint8)
    gu_row, d_row = D // 64 * 36, F // 64 * 36
    tail = blob[-16:].view(np.float32).astype(np.float64)

    def mat(off, rows, cols, row_bytes):
        m = blob[off:off + rows * row_bytes].reshape(rows, cols // 64, 36)
        sc = e4m3_decode(m[:, :, 0:4])                       # [rows, blocks, 4]
        code = m[:, :, 4:].reshape(rows, cols // 64, 4, 8)  # [rows, blocks, sub, byte]
        lo = code & 15                                       # values 0..7 of the sub-block
        hi = code >> 4                                       # values 8..15
        vals = np.concatenate([e2m1_decode(lo), e2m1_decode(hi)], axis=3)   # [rows, blocks, sub, 16]
        vals = vals * sc[:, :, :, None]
        return vals.reshape(rows, cols)

    gate = mat(0, F, D, gu_row) * tail[0]
    up = mat(F * gu_row, F, D, gu_row) * tail[1]
    down = mat(2 * F * gu_row, D, F, d_row) * tail[2]
    return gate, up, down


def f16_bits_to_f64(h):
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float64)


def bf16_bits_to_f64(h):
    u = np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16
    return u.view(np.float32).astype(np.float64)


def q8_dense(codes, scales, rows, cols):
    c = np.asarray(codes, dtype=np.int8).reshape(rows, cols // 32, 32).astype(np.float64)
    s = f16_bits_to_f64(np.asarray(scales).reshape(rows, cols // 32))
    return (c * s[:, :, None]).reshape(rows, cols)


def dequant(q, s, group):
    q = np.asarray(q, dtype=np.int8).astype(np.float64)
    s = np.asarray(s, dtype=np.float32).astype(np.float64)
    return (q.reshape(-1, group) * s.reshape(-1, 1)).reshape(q.shape)
