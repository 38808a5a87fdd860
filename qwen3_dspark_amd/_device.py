"""Device selection and per-device reusable buffers for the HIP path."""
import torch

ARCH = 'gfx950'


def require_gfx950(device):
    """Canonical torch.device of an explicitly selected gfx950 GPU, else raise.

    There is no CPU or non-gfx950 path: callers fail loudly instead.
    """
    device = torch.device(device)
    if device.type != 'cuda' or torch.version.hip is None or not torch.cuda.is_available():
        raise RuntimeError('The MI355X HIP path requires an explicitly selected ROCm gfx950 GPU; no CPU fallback')
    if device.index is None:
        device = torch.device('cuda', torch.cuda.current_device())
    arch = getattr(torch.cuda.get_device_properties(device), 'gcnArchName', '') or ''
    if arch.split(':')[0] != ARCH:
        raise RuntimeError(f'The MI355X HIP path requires a {ARCH} GPU, found {arch!r}')
    return device


class Workspace:
    """Grow-only device scratch (uint8) reused across calls on one device."""

    def __init__(self, device):
        self.device = device
        self._buf = None

    def get(self, nbytes):
        nbytes = max(int(nbytes), 16)
        if self._buf is None or self._buf.numel() < nbytes:
            self._buf = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
        return self._buf

    @property
    def nbytes(self):
        return 0 if self._buf is None else self._buf.numel()
