"""GPU check of the measurement helper ss_hbm_read_probe: every byte of the buffer is
read (the XOR of the per-workgroup words equals the XOR of the buffer's 32-bit words,
computed on the host), at grid sizes below and above the buffer's 4 KiB chunk count."""

import numpy as np
import pytest
import torch

from soupsuck_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes, blocks", [(16, 1), (4096 * 3 + 48, 2), (1 << 20, 256),
                                            (33_947_648, 1024)])
def test_read_probe_reads_every_word(device, nbytes, blocks):
    gen = torch.Generator(device="cpu").manual_seed(nbytes)
    host = torch.randint(0, 256, (nbytes,), generator=gen, dtype=torch.uint8)
    buf = host.to(device)
    sink = torch.empty(blocks, device=device, dtype=torch.int32)
    _lib.call("ss_hbm_read_probe", buf.data_ptr(), nbytes, blocks, sink.data_ptr(),
              _lib.stream(device))
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(host.numpy().view(np.uint32))
    assert int(got) == int(want)
