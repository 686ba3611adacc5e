"""Device helpers for the GPU tests (torch for device memory only)."""
import ctypes as C

import numpy as np
import torch

import sp_hip as S


def dev(a):
    """numpy -> contiguous cuda tensor (same dtype; uint16 fp16 bits go as int16)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    if a.dtype == np.uint8:
        return torch.from_numpy(a).cuda()
    return torch.from_numpy(a).cuda()


def host(t, dtype=None):
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def p(t):
    return C.c_void_p(t.data_ptr())


def stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def empty_u8(n):
    return torch.zeros(n, dtype=torch.uint8, device="cuda")


def empty_f32(*shape):
    return torch.zeros(*shape, dtype=torch.float32, device="cuda")


def empty_f16(*shape):
    return torch.zeros(*shape, dtype=torch.int16, device="cuda")


def order_dev(hd):
    import oracle_py as O
    return dev(O.mobius_order(hd).astype(np.int32))


def encode(bc, order_t, src_t, dtype, n, hd, norm=S.NORM_FINAL, generic=False, dst=None):
    """[n, hd] contiguous -> [n, B] records through sp_hip_ship_encode(_generic)."""
    out = dst if dst is not None else empty_u8(n * bc.total_bytes)
    fn = S.lib().sp_hip_ship_encode_generic if generic else S.lib().sp_hip_ship_encode
    rc = fn(C.byref(bc), p(order_t) if order_t is not None else None, norm, p(src_t), dtype, 0, hd,
            p(out), 0, 1, n, stream())
    S.check(rc, "encode")
    return out


def decode(bc, order_t, rec_t, dtype, n, hd, norm=S.NORM_FINAL, max_bands=-1, generic=False):
    out = empty_f32(n * hd) if dtype == S.DTYPE_F32 else empty_f16(n * hd)
    fn = S.lib().sp_hip_ship_decode_generic if generic else S.lib().sp_hip_ship_decode
    rc = fn(C.byref(bc), p(order_t) if order_t is not None else None, norm, max_bands, p(rec_t), 0,
            p(out), dtype, 0, hd, 1, n, stream())
    S.check(rc, "decode")
    return out


_hip = None


def d2h(dptr, n):
    """Copy n bytes from a raw device pointer owned by the library to a numpy array."""
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    torch.cuda.synchronize()
    out = np.empty(n, dtype=np.uint8)
    rc = _hip.hipMemcpy(out.ctypes.data, dptr, n, 2)  # hipMemcpyDeviceToHost
    assert rc == 0, rc
    return out
