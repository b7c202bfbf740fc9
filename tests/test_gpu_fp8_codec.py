"""The device E4M3 encoder (clamp + v_cvt_pk_fp8_f32, what ROCm's
__hip_cvt_float_to_fp8(x, SATFINITE, E4M3) lowers to on gfx950 and the append
kernel uses) equals the oracle's encoder on every finite float32; the device
decoder (v_cvt_scalef32_pk_bf16_fp8) equals the oracle's decoder on all 256 codes."""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import oracle
import phaseshift_amd as P

pytestmark = pytest.mark.gpu


def test_device_decode_all_codes(dev):
    out = torch.zeros(256, dtype=torch.float32, device=dev)
    P.check("decode", P.lib().psk_selftest_e4m3_decode_all(out.data_ptr(), None))
    torch.cuda.synchronize()
    want = oracle.e4m3_decode(np.arange(256, dtype=np.uint8))
    got = out.cpu().numpy()
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[~fin]))


def test_device_encode_every_finite_float(dev):
    CH = 1 << 27
    L = oracle.lib()
    buf = torch.empty(CH // 4, dtype=torch.int32, device=dev)
    bad = 0
    with ThreadPoolExecutor(8) as ex:
        for i in range(1 << 5):
            P.check("encode", P.lib().psk_selftest_e4m3_encode_range(i * CH, CH, buf.data_ptr(),
                                                                      None))
            got = buf.cpu().numpy().view(np.uint8)
            parts = np.array_split(np.arange(CH, dtype=np.int64), 8)

            def job(ix):
                want = np.empty(len(ix), np.uint8)
                L.or_e4m3_encode_range(i * CH + int(ix[0]), len(ix), want)
                x = (np.arange(len(ix), dtype=np.uint64) + i * CH + int(ix[0])).astype(np.uint32)
                f = x.view(np.float32)
                fin = np.isfinite(f)
                return int(np.count_nonzero(got[ix[0]:ix[0] + len(ix)][fin] != want[fin]))

            bad += sum(ex.map(job, parts))
    assert bad == 0
