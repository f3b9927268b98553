"""Writes tests/golden/sr_bf16_reference.npz: fp32 inputs and their stochastically rounded bf16 outputs,
checked against the reference's own rounding rule.

The reference defines the rounding only inside its test helper
`assert_stochastic_bf16_matches_fp32` (tests/utils.py:70-92 of the reference), which computes the
expected bf16 bits from the fp32 output and asserts that the kernel's output equals them.  This script
imports that helper from the reference checkout (it needs numpy and torch only), feeds it this
repository's oracle output (oracle/epilogue.py: stochastic_round_bf16) for each input, and writes the
fixture only if the reference's helper accepts every case: the stored outputs are then the reference's
own.  Run in a container that holds the reference: `python tests/golden/make_sr_golden.py [ref_root]`.
The fixture is data (inputs, expected bits); no reference code is stored.
"""
import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import epilogue as oe  # noqa: E402


def _cases():
    g = torch.Generator().manual_seed(2024)
    out = []
    for shape in ((4, 16), (3, 10), (2, 5, 7), (1, 1), (8, 33), (2, 130)):   # ragged rows: zero-padded quartets
        x = torch.randn(shape, generator=g) * torch.exp2(torch.randint(-20, 20, shape, generator=g).float())
        out.append(x)
    x = torch.tensor([[float('nan'), float('inf'), -float('inf'), 0.0, -0.0, 1e-40, -1e-40, 3.3895314e38,
                       -3.3895314e38, 1.0, 1.0 + 2 ** -8, 1.0 + 2 ** -17]])
    out.append(x)
    bits = torch.randint(0, 2 ** 31 - 1, (6, 24), generator=g, dtype=torch.int64)
    sign = torch.randint(0, 2, (6, 24), generator=g, dtype=torch.int64) << 31
    out.append(((bits | sign) & 0xffffffff).to(torch.int64).numpy().astype(np.uint32).view(np.float32))
    return [torch.as_tensor(np.asarray(c, dtype=np.float32)) for c in out]


def main(ref_root='/root/reference'):
    spec = importlib.util.spec_from_file_location('reference_test_utils', os.path.join(ref_root, 'tests', 'utils.py'))
    ref = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(ref)
    arrays = {}
    for i, x in enumerate(_cases()):
        ours = oe.stochastic_round_bf16(x)
        ref.assert_stochastic_bf16_matches_fp32(ours, lambda fp32, x=x: fp32.copy_(x), f'case {i}')
        arrays[f'x{i}'] = x.numpy().view(np.uint32)
        arrays[f'y{i}'] = ours.view(torch.int16).numpy().view(np.uint16)
    path = os.path.join(HERE, 'sr_bf16_reference.npz')
    np.savez_compressed(path, **arrays)
    print(f'wrote {path}: {len(arrays) // 2} cases, all accepted by the reference helper')


if __name__ == '__main__':
    main(*sys.argv[1:])
