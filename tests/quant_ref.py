"""fp64 dequantisation of the reference's weight formats, written from the
format descriptions (src/gguf.h:46-135) with numpy array operations, as an
independent check of the oracle's matmul (not a copy of its loops)."""
import numpy as np

F32, F16, Q4_0, Q8_0, Q6_K = 0, 1, 2, 8, 14


def _f16(b):
    return np.ascontiguousarray(b).view(np.float16)[..., 0].astype(np.float64)


def dequant(raw: np.ndarray, wtype: int, rows: int, cols: int) -> np.ndarray:
    """[rows][cols] float64 weights from the raw GGUF bytes."""
    raw = np.ascontiguousarray(raw, np.uint8)
    if wtype == F32:
        return raw.view(np.float32).reshape(rows, cols).astype(np.float64)
    if wtype == F16:
        return raw.view(np.float16).reshape(rows, cols).astype(np.float64)
    if wtype == Q8_0:
        b = raw.reshape(rows, cols // 32, 34)
        d = _f16(b[..., 0:2])
        qs = b[..., 2:34].view(np.int8).astype(np.float64)
        return (d[..., None] * qs).reshape(rows, cols)
    if wtype == Q4_0:
        b = raw.reshape(rows, cols // 32, 18)
        d = _f16(b[..., 0:2])
        qs = b[..., 2:18].astype(np.int64)
        # element j: low nibble of byte j; element 16 + j: high nibble; both minus 8
        q = np.concatenate([(qs & 15) - 8, (qs >> 4) - 8], axis=-1).astype(np.float64)
        return (d[..., None] * q).reshape(rows, cols)
    if wtype == Q6_K:
        b = raw.reshape(rows, cols // 256, 210)
        ql = b[..., 0:128].astype(np.int64)
        qh = b[..., 128:192].astype(np.int64)
        sc = b[..., 192:208].view(np.int8).astype(np.float64)
        d = _f16(b[..., 208:210])
        out = np.empty((rows, cols // 256, 256))
        for h in range(2):          # two halves of 128 weights
            lq = ql[..., 64 * h: 64 * h + 64]   # 64 bytes of low nibbles
            hq = qh[..., 32 * h: 32 * h + 32]   # 32 bytes, 2 bits per weight
            for k in range(4):      # 4 runs of 32 weights sharing hq
                low = (lq[..., 32 * (k & 1): 32 * (k & 1) + 32] >> (4 * (k >> 1))) & 15
                q = (low | (((hq >> (2 * k)) & 3) << 4)) - 32           # [rows, nb, 32]
                # the run's 32 weights use scales sc[8h + 2k] (first 16) and sc[8h + 2k + 1]
                s = np.repeat(sc[..., 8 * h + 2 * k: 8 * h + 2 * k + 2], 16, axis=-1)
                out[..., 128 * h + 32 * k: 128 * h + 32 * k + 32] = d[..., None] * s * q
        return out.reshape(rows, cols)
    raise ValueError(wtype)


def matmul_f64(raw, x, wtype, rows, cols):
    """(W.x in float64, sum_j |w_ij x_j|) per row."""
    w = dequant(raw, wtype, rows, cols)
    x = np.asarray(x, np.float64)
    return w @ x, np.abs(w) @ np.abs(x)
