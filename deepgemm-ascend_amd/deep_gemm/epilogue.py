"""GEMM epilogue classes (the reference's ``deep_gemm.epilogue`` submodule,
csrc/apis/epilogue_class.hpp:10-20 and csrc/jit_kernels/epilogue_class.hpp:14-128).

Identity and Alpha run in the GEMM kernels' register epilogue.  FP8Quantization and
BF16StochasticRounding exist so that code naming them imports, but this build rejects
them at call time (they are outside the hot path this library implements).
"""


class Epilogue:
    def check(self, c, d) -> None:
        import torch
        if d.dtype not in (torch.bfloat16, torch.float32):
            raise RuntimeError('Assertion error: D must be bf16 or fp32')


class Identity(Epilogue):
    pass


class Alpha(Epilogue):
    def __init__(self, alpha: float):
        self.alpha = float(alpha)


class FP8Quantization(Epilogue):
    def __init__(self, sfd):
        self.sfd = sfd

    def check(self, c, d) -> None:
        raise RuntimeError('FP8Quantization epilogue is not supported by the MI355X build')


class BF16StochasticRounding(Epilogue):
    def check(self, c, d) -> None:
        raise RuntimeError('BF16StochasticRounding epilogue is not supported by the MI355X build')


class _Bias(Epilogue):
    def __init__(self, bias):
        self.bias = bias


def resolve(epilogue, c, d, alpha=None):
    """csrc/jit_kernels/epilogue_class.hpp:110-128: epilogue class and alpha are exclusive."""
    if (epilogue is not None) + (alpha is not None) > 1:
        raise RuntimeError('The epilogue class, alpha and the FP8 output pair are exclusive')
    resolved = epilogue
    if alpha is not None:
        resolved = Alpha(alpha)
    elif resolved is None:
        resolved = Identity()
    resolved.check(c, d)
    return resolved
