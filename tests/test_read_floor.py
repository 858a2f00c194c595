"""oxs_read_floor, the diagnostic read of the stream phase's access pattern:
each (row, 8192-logit chunk) block writes the largest bit pattern of its
chunk, checked against numpy on a ragged shape."""
import ctypes

import numpy as np
import pytest

from oxide_sampler import _abi


@pytest.mark.gpu
def test_read_floor_sinks_each_chunk(torch_gpu):
    t = torch_gpu
    lib = _abi.load_library()
    B, V, ld = 5, 20004, 20008  # three chunks per row, the last one short; a padded row stride
    rng = np.random.default_rng(3)
    x = rng.standard_normal((B, ld)).astype(np.float32)
    d = t.from_numpy(x).cuda()
    S = (V + 8191) // 8192
    sink = t.zeros(B * S, dtype=t.int32, device="cuda")
    print(f"\n[case] oxs_read_floor B={B} V={V} ld={ld}", flush=True)
    _abi.check(lib.oxs_read_floor(ctypes.c_void_p(d.data_ptr()), V, ld, B, ctypes.c_void_p(sink.data_ptr()), None),
               "oxs_read_floor")
    t.cuda.synchronize()
    bits = x.view(np.uint32)[:, :V]
    want = np.array([bits[b, c * 8192:min((c + 1) * 8192, V)].max() for b in range(B) for c in range(S)], np.uint32)
    np.testing.assert_array_equal(sink.cpu().numpy().view(np.uint32), want)
    assert lib.oxs_read_floor(ctypes.c_void_p(d.data_ptr()), 20002, ld, B, ctypes.c_void_p(sink.data_ptr()),
                              None) == _abi.OXS_ERR_INVALID_ARGUMENT  # vocab not a multiple of 4
