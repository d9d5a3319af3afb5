"""Matrix arguments of the octex library: numpy arrays, torch tensors (host or GPU), and arrays of any other
framework that exports DLPack or __cuda_array_interface__, seen as one of two things the C ABI takes: a numpy
array (host memory) or a torch tensor (host or device memory).  Device operands carry the HIP stream their
producer is ordered on, so that the library's work waits for it and the results are ordered on it; results
go back to the caller in the framework of the operand.

Only numpy is required.  torch is imported when a device operand or a torch tensor is given; other frameworks
are reached through the module their array belongs to (sys.modules), never imported here.
"""

import sys

import numpy as np

# __cuda_array_interface__ (version 3) stream codes: 1 the legacy default stream, 2 the per-thread one
_CAI_LEGACY, _CAI_PER_THREAD = 1, 2
_HIP_NULL_STREAM, _HIP_PER_THREAD_STREAM = 0, 2


def _module_of(a):
    return type(a).__module__.partition(".")[0]


def is_torch(a):
    return _module_of(a) == "torch"


def is_foreign_device(a):
    """An array of another framework (CuPy, JAX, ...) with DLPack or __cuda_array_interface__."""
    return (not isinstance(a, np.ndarray) and not is_torch(a)
            and (hasattr(a, "__cuda_array_interface__") or hasattr(a, "__dlpack__")))


def _hip_stream_of_cai(code):
    """The HIP stream of a __cuda_array_interface__ 'stream' entry (None: the producer needs no ordering)."""
    if code is None:
        return None
    code = int(code)
    return {_CAI_LEGACY: _HIP_NULL_STREAM, _CAI_PER_THREAD: _HIP_PER_THREAD_STREAM}.get(code, code)


def _foreign_stream(a):
    """The stream a foreign device array was produced on: the interface's own 'stream' entry, else the current
    stream of its framework when the framework has that notion (CuPy), else the null stream."""
    cai = getattr(a, "__cuda_array_interface__", None)
    if cai is not None and "stream" in cai:
        s = _hip_stream_of_cai(cai["stream"])
        return _HIP_NULL_STREAM if s is None else s
    mod = sys.modules.get(_module_of(a))
    cuda = getattr(mod, "cuda", None)
    get = getattr(cuda, "get_current_stream", None)
    if callable(get):
        return int(get().ptr)
    return _HIP_NULL_STREAM


class Operand:
    """One matrix argument: `value` is what crosses the C ABI (numpy or torch), `stream` the HIP stream a device
    operand is ordered on (None for host memory), `origin` the caller's object."""

    def __init__(self, value, origin, stream=None):
        self.value = value
        self.origin = origin
        self.stream = stream

    @property
    def shape(self):
        return tuple(int(v) for v in self.value.shape)

    @property
    def on_device(self):
        return self.stream is not None

    @property
    def device(self):
        return self.value.device if self.on_device else None

    def new(self, rows, cols, dtype):
        """An output of the operand's kind: numpy for host operands, a torch tensor on its device otherwise."""
        if not self.on_device:
            return np.empty((rows, cols), dtype)
        torch = sys.modules["torch"]
        return torch.empty((rows, cols), dtype=getattr(torch, np.dtype(dtype).name), device=self.value.device)

    def respond(self, result):
        """A result (numpy or torch) in the framework of the operand's origin: numpy for numpy and other host
        inputs, torch for torch tensors (host results of host tensors as torch CPU tensors), the origin
        framework's from_dlpack for foreign device arrays."""
        if is_torch(self.origin):
            torch = sys.modules["torch"]
            return torch.from_numpy(result) if isinstance(result, np.ndarray) else result
        if is_foreign_device(self.origin):
            conv = getattr(sys.modules.get(_module_of(self.origin)), "from_dlpack", None)
            return conv(result) if conv is not None else result
        return result


def operand(a, dtypes=(np.float32,), name="queries"):
    """The matrix `a` prepared for the C ABI: dense row major, of the first of `dtypes` unless it already has one
    of them, in the memory where it lies.  A vector is one row."""
    want = tuple(np.dtype(t) for t in dtypes)
    if is_foreign_device(a):
        import torch

        stream = _foreign_stream(a)
        t = torch.from_dlpack(a) if hasattr(a, "__dlpack__") else torch.as_tensor(a, device="cuda")
        return _torch_operand(t, a, want, name, stream)
    if is_torch(a):
        return _torch_operand(a, a, want, name, None)
    x = np.asarray(a)
    if x.ndim == 1:
        x = x[None, :]
    if x.ndim != 2:
        raise ValueError(f"octex: {name} must be a matrix [m, dim]")
    if x.dtype not in want:
        x = x.astype(want[0])
    return Operand(np.ascontiguousarray(x), a)


def _torch_operand(t, origin, want, name, stream):
    torch = sys.modules["torch"]
    t = t.detach()
    if t.ndim == 1:
        t = t[None, :]
    if t.ndim != 2:
        raise ValueError(f"octex: {name} must be a matrix [m, dim]")
    have = str(t.dtype).replace("torch.", "")
    if have not in [w.name for w in want]:
        t = t.to(getattr(torch, want[0].name))
    t = t.contiguous()
    if t.device.type == "cpu":
        return Operand(t.numpy(), origin)
    if t.device.type != "cuda":
        raise TypeError(f"octex: {name} must lie in host or GPU memory, not on {t.device}")
    if stream is None:
        stream = int(torch.cuda.current_stream(t.device).cuda_stream)
    return Operand(t, origin, stream)


def shape_of(a):
    """The shape of an array of any supported framework (a DLPack-only array through a torch view)."""
    if hasattr(a, "shape"):
        return tuple(int(v) for v in a.shape)
    cai = getattr(a, "__cuda_array_interface__", None)
    if cai is not None:
        return tuple(int(v) for v in cai["shape"])
    import torch

    return tuple(int(v) for v in torch.from_dlpack(a).shape)


def write_into(dst, src):
    """Copy the result src (numpy or torch) into the caller's array dst (numpy, torch or foreign), converting
    the element type as numpy's / torch's assignment does."""
    if isinstance(dst, np.ndarray):
        dst[...] = src.cpu().numpy() if is_torch(src) else src
        return dst
    import torch

    view = dst if is_torch(dst) else (torch.from_dlpack(dst) if hasattr(dst, "__dlpack__")
                                      else torch.as_tensor(dst, device="cuda"))
    view.copy_(src if is_torch(src) else torch.from_numpy(np.ascontiguousarray(src)))
    return dst


def host_rows(a, dtypes=(np.float32, np.float16), name="vectors"):
    """A host copy (numpy, dense, row major) of a matrix from any framework, for data kept on the host."""
    op = operand(a, dtypes, name)
    v = op.value
    return v.cpu().numpy() if op.on_device else v
