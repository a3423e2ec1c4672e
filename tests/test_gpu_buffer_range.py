"""The hardware rule the kernels' bounds handling rests on (needs an MI355X).

Every K, V, scale and split-partial load of the attention kernels goes
through a raw buffer descriptor that ends at the last valid byte, and the
kernels rely on loads past that end returning zeros (masked tokens, splits
past S, a 16-byte scale load that crosses the end of a row). The probe reads
a 64-dword descriptor over a larger buffer filled with i + 1 (so a load that
the range check let through would return a nonzero value, from memory that
is still inside the allocation) and checks each way an offset can reach past
the end: in the VGPR offset, the SGPR offset and the immediate field, and a
16-byte load that straddles the end, whose dwords are checked one by one."""

import ctypes

import pytest
import torch

import fqkv_decode

pytestmark = pytest.mark.gpu

VP = ctypes.c_void_p


def test_raw_buffer_loads_past_num_records_read_zero():
    L = ctypes.CDLL(fqkv_decode.lib_path())
    L.fqkv_last_error.restype = ctypes.c_char_p
    L.fqkv_probe_buffer_range.argtypes = [VP, ctypes.c_size_t, ctypes.c_int, VP, VP]
    records = 256
    buf = torch.arange(1, 1025, dtype=torch.int32, device="cuda")  # dword i holds i + 1
    out = torch.full((16,), -1, dtype=torch.int32, device="cuda")
    rc = L.fqkv_probe_buffer_range(buf.data_ptr(), buf.numel() * 4, records, out.data_ptr(),
                                   torch.cuda.current_stream().cuda_stream)
    assert rc == 0, L.fqkv_last_error().decode()
    got = out.cpu().tolist()
    last = records // 4  # value of the last dword in range
    assert got[0] == last, "in-range load"
    assert got[1] == 0, "VGPR offset past the end"
    assert got[2] == 0, "SGPR offset past the end"
    assert got[3] == 0, "SGPR offset alone past the end"
    assert got[4] == 0, "immediate offset past the end"
    assert got[5:9] == [last - 1, last, 0, 0], "16-byte load straddling the end: per-dword zeros"
    assert got[9:] == [-1] * 7, "the probe writes nine dwords"

