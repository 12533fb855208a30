import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(REPO, "codon-infer_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))

GOLDEN = os.path.join(REPO, "tests", "golden")
# The shipped 8M FP32 weights (grouped_canonical_v1).  build() copies the
# reference's file here (git-ignored) so that GPU runs see it too.
WEIGHTS_8M_CANDIDATES = [os.path.join(GOLDEN, "data", "esm2_8m_weights.bin"),
                         "/root/reference/esm2_8m_weights.bin"]
PEPTIDE = "AQVGDSGGPMLCNGQLQGVTSWGYVCAQPEYPGVYTEVS"  # test_peptidase.fasta
AA_ORDER = "LAGVSERTIDPKQNFYMHWC"  # token ids 4..23


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libcodon_hip.so on the GPU)")


def weights_8m_path():
    for p in WEIGHTS_8M_CANDIDATES:
        if os.path.exists(p) and os.path.getsize(p) == 30_091_652:
            return p
    return None


@pytest.fixture(scope="session")
def w8m_path():
    p = weights_8m_path()
    if p is None:
        pytest.skip("shipped 8M weights not present")
    return p


def decode(ids):
    return "".join(AA_ORDER[i - 4] if 4 <= i <= 23 else "?" for i in ids)
