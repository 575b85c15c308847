"""The read probe (tb_read_probe) that bench.py uses for the GEMVs' read
ceiling: every byte of the buffer is read exactly once, for every grid shape
the benchmark tries and for sizes that leave a partial last pass."""
import ctypes as C

import numpy as np
import pytest
import torch

from torchburn_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [(1 << 20) + 48, 36700160])
@pytest.mark.parametrize("blocks,loads", [(512, 4), (768, 4), (1024, 8), (1536, 4), (2048, 8),
                                          (3, 16)])
def test_read_probe_reads_every_byte_once(nbytes, blocks, loads):
    print(f"case read probe bytes={nbytes} blocks={blocks} loads={loads}", flush=True)
    g = np.random.default_rng(nbytes + blocks)
    host = g.integers(0, 1 << 32, nbytes // 4, dtype=np.uint32)
    buf = torch.from_numpy(host.view(np.int32)).cuda()
    out = torch.zeros(blocks * 256, dtype=torch.int32, device="cuda")
    got = C.c_int64(0)
    _lib.call("tb_read_probe", buf.data_ptr(), nbytes, blocks, loads, out.data_ptr(),
              C.addressof(got), None)
    torch.cuda.synchronize()
    assert got.value == nbytes & ~15
    # each 16-byte piece is loaded by one thread and xor-folded into its word
    fold = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(host[: got.value // 4])
    assert fold == want
