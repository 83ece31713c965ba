"""State shared by the patches during one training step (solution/_state.py:4-25)."""


class _State:
    def __init__(self):
        self.request = False
        self.stats = None
        self.packing = None
        self.packing_active = False
        self.norm_link = None


STATE = _State()


def on_gpu(tensor):
    """The HIP kernels take GPU tensors only; everything else takes the original code path."""
    return tensor.is_cuda
