"""GPU: emrs_xor_checksum, the read-only pass over a device buffer (its XOR of 32-bit words)."""

import numpy as np
import pytest
import torch

from elasticmegatron_amd import _native

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [0, 16, 4096 + 16, (1 << 20) + 48, 3 * (32 << 10) * 1280 + 32])
def test_xor_checksum_matches_numpy(gpu_device, nbytes):
    """Sizes below one chunk, ragged tails, and more chunks than the grid has workgroups."""
    rng = np.random.default_rng(nbytes)
    words = rng.integers(0, 2 ** 32, nbytes // 4 + 4, dtype=np.uint32)
    buf = torch.from_numpy(words.view(np.int32)).to(gpu_device)
    out = torch.full((1,), -1, dtype=torch.int32, device=gpu_device)   # zeroed by the call
    print(f"case xor checksum {nbytes} B", flush=True)
    _native.xor_checksum(buf.data_ptr(), nbytes, out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    want = np.bitwise_xor.reduce(words[:nbytes // 4]) if nbytes else np.uint32(0)
    assert int(out.cpu().numpy().view(np.uint32)[0]) == int(want)
