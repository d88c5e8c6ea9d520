"""The bounded split-K wait's error path, forced from the host.

A combine's last block waits (bounded) for each partner's mailbox slot. A wait that gives up
must surface as an error, not as a silently wrong sum. The test drives the device's slot wait
through w4a16_debug_slot_wait on a slot the host never writes (its bound of 16 polls ends the
wait, so the kernel exits normally), then requires w4a16_split_wait_status to report it once and
to be clean afterwards; a written slot is taken with its value and cleared, with no error."""

import struct

import numpy as np
import pytest

import w4a16


@pytest.mark.gpu
def test_split_wait_timeout_reported(cuda):
    import torch

    w4a16.split_wait_status()          # clean before
    slot = torch.zeros(2, dtype=torch.int64, device=cuda)
    out = torch.full((4,), 7.0, dtype=torch.float32, device=cuda)
    stream = torch.cuda.current_stream().cuda_stream
    print("unwritten slot, 16 polls", flush=True)
    assert lib_call(slot, 16, out, stream) == 0
    torch.cuda.synchronize()
    assert out[0].item() == 0.0
    with pytest.raises(w4a16.W4A16Error, match="gave up"):
        w4a16.split_wait_status()
    w4a16.split_wait_status()          # the count was cleared by the report

    value = 3.5
    bits = struct.unpack("<I", struct.pack("<f", value))[0]
    slot[0] = (1 << 32) | bits
    print("written slot", flush=True)
    assert lib_call(slot, 16, out, stream) == 0
    torch.cuda.synchronize()
    assert out[0].item() == value
    assert slot[0].item() == 0         # taken slots are cleared for the next call
    w4a16.split_wait_status()


def lib_call(slot, polls, out, stream):
    return w4a16.lib.w4a16_debug_slot_wait(slot.data_ptr(), polls, out.data_ptr(), stream)


def test_status_symbols_exported():
    assert hasattr(w4a16.lib, "w4a16_split_wait_status")
    assert hasattr(w4a16.lib, "w4a16_debug_slot_wait")
    assert np.int32(w4a16.W4A16_ERR_HIP) == -1
