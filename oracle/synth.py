"""numpy restatement of the seeded synthetic generator (test infrastructure).

value(seed, param, kind, full flat index):
  key  = mix64(mix64(seed + G) + (4*param + stream + 1) * G)
  h    = mix64(key + (index + 1) * G)
  s    = sum of the four 16-bit lanes of h - 131070
  v    = float32(s) * scale[stream]          (one fp32 rounding)
  stream 0: param = bf16 round-to-nearest-even of v, main = its exact upcast
  stream 1: exp_avg = v; stream 2: exp_avg_sq = |v|
"""

import numpy as np

G = 0x9E3779B97F4A7C15
M64 = (1 << 64) - 1
SCALE_BITS = (0x350DE3BD, 0x32E305FB, 0x2DE878D0)  # 0.02, 1e-3, 1e-6 divided by 37837.227


def _mix_int(z: int) -> int:
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _mix_arr(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def stream_key(seed: int, param_id: int, stream: int) -> int:
    return _mix_int((_mix_int((seed + G) & M64) + (4 * param_id + stream + 1) * G) & M64)


def f32_bits(seed: int, param_id: int, stream: int, idx: np.ndarray) -> np.ndarray:
    """uint32 bits of the stream's fp32 value at full flat indices ``idx`` (before bf16 rounding)."""
    key = np.uint64(stream_key(seed, param_id, stream))
    i = np.asarray(idx, dtype=np.uint64)
    with np.errstate(over="ignore"):
        h = _mix_arr(key + (i + np.uint64(1)) * np.uint64(G))
    m = np.uint64(0xFFFF)
    s = ((h & m) + ((h >> np.uint64(16)) & m) + ((h >> np.uint64(32)) & m) + (h >> np.uint64(48))).astype(np.int64)
    v = (s - 131070).astype(np.float32) * np.array(SCALE_BITS[stream], dtype=np.uint32).view(np.float32)
    bits = v.astype(np.float32).view(np.uint32)
    if stream == 2:
        bits = bits & np.uint32(0x7FFFFFFF)
    return bits


def bf16_round(bits: np.ndarray) -> np.ndarray:
    """uint16 bits of the bf16 nearest-even rounding of fp32 ``bits`` (finite inputs)."""
    b = bits.astype(np.uint64)
    return ((b + 0x7FFF + ((b >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)).astype(np.uint16)


_KIND_CODE = {"param": 0, "main": 1, "exp_avg": 2, "exp_avg_sq": 3}
_clib = None


def _c_library():
    """oracle/build/libsynth_ref.so (oracle/Makefile) when it has been built, else None."""
    global _clib
    if _clib is None:
        import ctypes
        import os

        path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "build", "libsynth_ref.so")
        if not os.path.exists(path):
            _clib = False
            return None
        lib = ctypes.CDLL(path)
        lib.oracle_synth.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p,
                                     ctypes.c_uint64, ctypes.c_void_p]
        _clib = lib
    return _clib or None


def values(seed: int, param_id: int, kind: str, idx: np.ndarray) -> np.ndarray:
    """kind in {param, main, exp_avg, exp_avg_sq}: bf16 returned as uint16 bits, fp32 as float32.

    Uses the C restatement when it is built (same definition, much faster);
    tests/test_synth.py checks that the two agree bit for bit.
    """
    lib = _c_library()
    if lib is not None:
        i = np.ascontiguousarray(idx, dtype=np.uint64)
        out = np.empty(i.size, dtype=np.uint32)
        lib.oracle_synth(seed & M64, param_id, _KIND_CODE[kind], i.ctypes.data, i.size, out.ctypes.data)
        return out.astype(np.uint16) if kind == "param" else out.view(np.float32)
    return values_numpy(seed, param_id, kind, idx)


def values_numpy(seed: int, param_id: int, kind: str, idx: np.ndarray) -> np.ndarray:
    """The numpy restatement (see ``values``)."""
    if kind in ("param", "main"):
        bf = bf16_round(f32_bits(seed, param_id, 0, idx))
        if kind == "param":
            return bf
        return (bf.astype(np.uint32) << np.uint32(16)).view(np.float32)
    stream = {"exp_avg": 1, "exp_avg_sq": 2}[kind]
    return f32_bits(seed, param_id, stream, idx).view(np.float32)
