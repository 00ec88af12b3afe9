"""Device/host plumbing for the GPU tests (numpy <-> torch CUDA tensors)."""
import numpy as np
import torch


def dev(a: np.ndarray) -> torch.Tensor:
    """Upload a numpy array (any dtype, viewed as bytes if needed) to cuda:0."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint64:
        a = a.view(np.int64)
    t = torch.from_numpy(a).cuda()
    torch.cuda.synchronize()  # the library runs on its own streams
    return t


def host(t: torch.Tensor, dtype) -> np.ndarray:
    return t.detach().cpu().numpy().view(dtype)


def zeros(n: int, dtype) -> torch.Tensor:
    tmap = {np.uint8: torch.uint8, np.uint16: torch.int16, np.uint32: torch.int32,
            np.float32: torch.float32, np.float64: torch.float64, np.int32: torch.int32}
    t = torch.zeros(n, dtype=tmap[dtype], device="cuda")
    torch.cuda.synchronize()
    return t


def sync():
    torch.cuda.synchronize()
