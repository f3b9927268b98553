"""GEMM epilogue classes (the reference's ``deep_gemm.epilogue`` submodule,
csrc/apis/epilogue_class.hpp:10-20 and csrc/jit_kernels/epilogue_class.hpp:14-128).

All of them run in the GEMM kernels' register epilogue: Identity and Alpha scale the fp32
accumulators, BF16StochasticRounding rounds each quartet of outputs with a hash of its own
fp32 bits, FP8Quantization writes e4m3 D plus per-(row, 32 columns) UE8M0 scales (``sfd``).
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
    """e4m3 output with UE8M0 scales per (row, 32 columns); ``sfd`` is int16 [M, B * N / 64],
    M-major (csrc/jit_kernels/epilogue_class.hpp:77-107)."""
    def __init__(self, sfd):
        self.sfd = sfd

    def check(self, c, d) -> None:
        import torch
        _check(c is None and d.dtype == torch.float8_e4m3fn, 'FP8 quantization requires a direct E4M3 output')
        _check(d.dim() in (2, 3))
        m, n = d.size(-2), d.size(-1)
        num_batches = d.size(0) if d.dim() == 3 else 1
        _check(n % 128 == 0, 'FP8 output requires N to be a multiple of 128')
        _check(d.stride(-1) == 1 and (d.dim() == 2 or d.stride(0) == n))
        sfd = self.sfd
        _check(sfd.dtype == torch.int16 and sfd.dim() == 2 and sfd.device == d.device)
        _check(sfd.size(0) == m and sfd.size(1) == num_batches * n // 64)
        _check((sfd.stride(0) == 1 or m == 1) and sfd.stride(1) == m)


class BF16StochasticRounding(Epilogue):
    """bf16 output rounded stochastically (csrc/jit_kernels/epilogue_class.hpp:66-75)."""
    def check(self, c, d) -> None:
        import torch
        _check(c is None and d.dtype == torch.bfloat16, 'Stochastic rounding requires a direct BF16 output')


def _check(cond: bool, msg: str = 'Assertion error') -> None:
    if not cond:
        raise RuntimeError(msg)


def resolve(epilogue, c, d, alpha=None, sfd=None):
    """csrc/jit_kernels/epilogue_class.hpp:110-128: epilogue class, alpha and the FP8 output
    pair's SF are exclusive."""
    if (epilogue is not None) + (alpha is not None) + (sfd is not None) > 1:
        raise RuntimeError('The epilogue class, alpha and the FP8 output pair are exclusive')
    resolved = epilogue
    if alpha is not None:
        resolved = Alpha(alpha)
    elif sfd is not None:
        resolved = FP8Quantization(sfd)
    elif resolved is None:
        resolved = Identity()
    resolved.check(c, d)
    return resolved
