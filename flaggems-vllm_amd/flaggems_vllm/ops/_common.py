"""Stream and device plumbing shared by the op wrappers."""
import contextlib

import torch


def current_stream_ptr(device: torch.device) -> int:
    """hipStream_t of torch's current stream on ``device`` (as an int)."""
    return torch.cuda.current_stream(device).cuda_stream


@contextlib.contextmanager
def on_device_of(t: torch.Tensor):
    """Make t's GPU the current HIP device for the launch, if it is not."""
    idx = t.device.index
    if idx is None or idx == torch.cuda.current_device():
        yield
    else:
        with torch.cuda.device(idx):
            yield
