"""`on_gpu`, the device test the patches use (the name the reference's tests replace to drive the
patched paths without a GPU, solution/_state.py:23-25)."""


def on_gpu(tensor):
    """The HIP kernels take GPU tensors only; everything else takes the original code path."""
    return tensor.is_cuda
