"""ctypes binding of oracle/_ref/libadi_backend.so: runs one adi::Backend entry
of the reference's cpu_backend() or of hip_backend() (adi_amd/backend) on
host arrays, through the reference's own dispatch table. Test helper."""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBRARY = os.path.join(ROOT, "oracle", "_ref", "libadi_backend.so")

CPU, HIP = 0, 1


class BackendError(Exception):
    def __init__(self, status, message):
        super().__init__(message)
        self.status = status  # 1: std::invalid_argument, 2: other
        self.message = message


def available() -> bool:
    return os.path.exists(LIBRARY)


_lib = None


def load():
    global _lib
    if _lib is None:
        _lib = C.CDLL(LIBRARY)
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _call(fn, *args):
    error = C.create_string_buffer(512)
    status = fn(*args, error, C.c_size_t(len(error)))
    if status != 0:
        raise BackendError(status, error.value.decode())


def name(which: int) -> str:
    out = C.create_string_buffer(128)
    status = load().bd_backend_name(C.c_int(which), out, C.c_size_t(len(out)))
    if status != 0:
        raise BackendError(status, out.value.decode())
    return out.value.decode()


def release_weights():
    _call(load().bd_release_weights)


def expert_matmul(which, m, x, batch, out_size=None, x_size=None):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(batch * m.rows if out_size is None else out_size, np.float32)
    _call(load().bd_expert_matmul, C.c_int(which), C.c_uint32(m.rows), C.c_uint32(m.columns),
          _p(m.trellis), C.c_size_t(m.trellis.size), _p(m.su_f16), C.c_size_t(m.su_f16.size),
          _p(m.sv_f16), C.c_size_t(m.sv_f16.size), _p(m.wave_gamma_f16),
          C.c_size_t(m.wave_gamma_f16.size), _p(m.tlut), _p(x),
          C.c_size_t(x.size if x_size is None else x_size), C.c_uint32(batch), _p(out),
          C.c_size_t(out.size))
    return out.reshape(-1, m.rows) if out_size is None else out


def ne_matmul(which, m, x, batch):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(batch * m.rows, np.float32)
    _call(load().bd_ne_matmul, C.c_int(which), C.c_uint32(m.rows), C.c_uint32(m.columns),
          _p(m.trellis), C.c_size_t(m.trellis.size), _p(m.su), _p(m.sv),
          C.c_float(m.weight_scale), _p(m.tlut), _p(x), C.c_size_t(x.size), C.c_uint32(batch),
          _p(out), C.c_size_t(out.size))
    return out.reshape(batch, m.rows)


def head_matmul(which, h, x, batch):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(batch * h.rows, np.float32)
    prot = h.protected_rows
    count = 0 if prot is None else prot.size
    _call(load().bd_head_matmul, C.c_int(which), C.c_uint32(h.rows), C.c_uint32(h.columns),
          _p(h.packed), _p(h.group_scale_f16), _p(prot), _p(h.protected_bf16),
          C.c_size_t(count), _p(x), C.c_size_t(x.size), C.c_uint32(batch), _p(out),
          C.c_size_t(out.size))
    return out.reshape(batch, h.rows)


def bf16_matmul(which, values, rows, columns, x, batch):
    x = np.ascontiguousarray(x, np.float32)
    values = np.ascontiguousarray(values, np.uint16)
    out = np.zeros(batch * rows, np.float32)
    _call(load().bd_bf16_matmul, C.c_int(which), C.c_uint32(rows), C.c_uint32(columns),
          _p(values), _p(x), C.c_size_t(x.size), C.c_uint32(batch), _p(out),
          C.c_size_t(out.size))
    return out.reshape(batch, rows)


def embedding_row(which, e, token, out_size=None):
    out = np.zeros(e.columns if out_size is None else out_size, np.float32)
    _call(load().bd_embedding_row, C.c_int(which), C.c_uint32(e.rows), C.c_uint32(e.columns),
          _p(e.packed), _p(e.minimum_f16), _p(e.maximum_f16), _p(e.exception_indexes),
          _p(e.exception_bf16), C.c_size_t(e.exception_indexes.size), C.c_uint32(token), _p(out),
          C.c_size_t(out.size))
    return out


def rms_norm(which, x, weight, offset, epsilon):
    x = np.ascontiguousarray(x, np.float32)
    weight = np.ascontiguousarray(weight, np.uint16)
    out = np.zeros_like(x)
    _call(load().bd_rms_norm, C.c_int(which), _p(x), _p(weight), C.c_size_t(x.size),
          C.c_float(offset), C.c_float(epsilon), _p(out))
    return out
