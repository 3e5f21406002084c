import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libttfa.so")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def tiny_config():
    """The reference's tiny model config (tests/conftest.py:8-20 of tinytrain)."""
    return dict(vocab_size=256, hidden_size=64, num_hidden_layers=2, num_attention_heads=4,
                num_key_value_heads=2, head_dim=64, intermediate_size=192, max_seq_len=32)

