import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs libfvs kernels)")


@pytest.fixture(scope="session")
def oracle_mod():
    from oracle import oracle as orc

    orc.lib()
    return orc


@pytest.fixture(scope="session")
def tiny(oracle_mod):
    """A small index built on the CPU: tables by the product's build code (torch on CPU), int8 codes by
    the oracle (the product computes them on the GPU)."""
    import torch

    from fanarvse_paper_amd import datagen, index

    N, d, NC = 6000, 256, 24
    X = datagen.gen(N, d, 16, 0.7, seed=0)
    Q = datagen.gen(48, d, 16, 0.7, seed=1, dtype=torch.float32)
    s1, code, _, _, Vr = index.build_index(X, nlist=NC, with_codes=False)
    Z, zs = oracle_mod.build_codes(X.numpy(), s1["order"].numpy(), s1["cell"].numpy(), s1["means16"].numpy(),
                                   Vr.numpy())
    idx = oracle_mod.index_from_tables(s1, code, Z, zs, Vr, X)
    GT = datagen.ground_truth(X, Q, 10).numpy()
    return dict(X=X, Q=Q, Qn=Q.numpy(), s1=s1, code=code, Vr=Vr, idx=idx, GT=GT)


def fp16_bits(a):
    return np.asarray(a, dtype=np.float16).view(np.uint16)
