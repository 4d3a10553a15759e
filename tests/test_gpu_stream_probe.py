"""GPU: the stream probe (mhcPreStreamProbe) reads and writes exactly the
bytes it is asked to.  Write block w (1 KB) holds the XOR of read block w's
four 1 KB lines, lane by lane (zeros past the read bytes), and nothing past
the write bytes changes; small grids make each wave take several blocks."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("read_kb,write_kb,workgroups", [(64, 16, 0), (16, 32, 0), (256, 64, 3),
                                                         (4, 1, 1)])
def test_stream_probe_output(pkg, device, read_kb, write_kb, workgroups):
    import torch

    rng = np.random.default_rng(read_kb * 7 + write_kb)
    guard = 8 << 10
    src_np = rng.integers(0, 2**32, (read_kb * 1024 + guard) // 4, dtype=np.uint32)
    src = torch.from_numpy(src_np.view(np.int32)).to(device)
    dst = torch.full(((write_kb * 1024 + guard) // 4,), 0x5A5A5A5A, dtype=torch.int32, device=device)
    print(f"[stream-probe] read {read_kb} KB write {write_kb} KB workgroups {workgroups}", flush=True)
    pkg.stream_probe(src, read_kb * 1024, dst, write_kb * 1024, workgroups)
    torch.cuda.synchronize()
    got = dst.cpu().numpy().view(np.uint32)
    blocks = src_np[: read_kb * 256].reshape(read_kb // 4, 4, 64, 4)
    want = np.bitwise_xor.reduce(blocks, axis=1).reshape(-1)  # 256 words per write block
    nw = write_kb * 256
    expect = np.zeros(nw, dtype=np.uint32)
    k = min(nw, want.size)
    expect[:k] = want[:k]
    np.testing.assert_array_equal(got[:nw], expect)
    assert (got[nw:] == 0x5A5A5A5A).all(), "bytes past the write size changed"
