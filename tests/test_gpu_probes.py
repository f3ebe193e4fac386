"""The float32 -> bfloat16 conversion every bfloat16 output takes (mbq_device.h bf16_bits: one v_cvt_pk_bf16_f32)
gives, on the device at hand, the bits of round-to-nearest-even with NaN kept quiet for every one of the 2^32 float32
inputs: mbq_probe_bf16 counts the inputs whose bits differ from that integer form, and the count must be zero."""
import ctypes

import pytest
import torch

from mashbox_amd import _lib as LIB

pytestmark = pytest.mark.gpu


def test_bf16_output_conversion_every_input():
    L = LIB.lib()
    diff = torch.zeros(2, dtype=torch.int64, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print("case: mbq_probe_bf16 over 2^32 float32 patterns", flush=True)
    LIB.check(L.mbq_probe_bf16(ctypes.c_void_p(diff.data_ptr()), st), "bf16 probe")
    torch.cuda.synchronize()
    assert diff.tolist() == [0, 0]
    with pytest.raises(LIB.MbqError):
        LIB.check(L.mbq_probe_bf16(None, st), "bf16 probe")
