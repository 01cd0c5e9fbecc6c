"""The allocation-free attention entry point (muyo_attention_decode_f16kv_static) against the
workspace entry point it shares its kernels with: bit-identical outputs on two calls in a row,
the second on a smaller shape (the fixed device array keeps the first call's partials, which the
second must not read), both also within 1e-3 of the oracle; shapes past the array are refused."""
import math

import numpy as np
import pytest

from conftest import close

pytestmark = pytest.mark.gpu


def _case(mh, torch, orc, heads, kv, hd, max_seq, pos, seed):
    lib = mh.load()
    s = torch.cuda.current_stream().cuda_stream
    kc = torch.empty(kv * max_seq * hd, dtype=torch.float16, device="cuda")
    vc = torch.empty_like(kc)
    mh.check(lib.muyo_fill_normal_f16(kc.data_ptr(), kc.numel(), seed, 0.0, 1.0, s))
    mh.check(lib.muyo_fill_normal_f16(vc.data_ptr(), vc.numel(), seed + 1, 0.0, 1.0, s))
    q = orc.normal_f32(heads * hd, seed + 2)
    qd = torch.from_numpy(q).cuda()
    pd = torch.tensor([pos], dtype=torch.int32, device="cuda")
    return lib, s, kc, vc, q, qd, pd


@pytest.mark.parametrize("order", ["large_then_small"])
def test_static_attention_matches_workspace_attention(mh, gpu, orc, order):
    torch = gpu
    cases = [(28, 4, 128, 2048, 2000, 71), (14, 2, 64, 256, 100, 81)]  # the second call is smaller
    for heads, kv, hd, max_seq, pos, seed in cases:
        print(f"[no-alloc] heads {heads} kv {kv} hd {hd} max_seq {max_seq} pos {pos}", flush=True)
        lib, s, kc, vc, q, qd, pd = _case(mh, torch, orc, heads, kv, hd, max_seq, pos, seed)
        scale = 1.0 / math.sqrt(hd)
        nbytes = lib.muyo_attention_decode_f16kv_workspace_bytes(heads, kv, hd, max_seq)
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        want = torch.empty_like(qd)
        got = torch.full_like(qd, float("nan"))
        mh.check(lib.muyo_attention_decode_f16kv(qd.data_ptr(), kc.data_ptr(), vc.data_ptr(), want.data_ptr(),
                                                 pd.data_ptr(), heads, kv, hd, max_seq, scale, ws.data_ptr(),
                                                 nbytes, s))
        mh.check(lib.muyo_attention_decode_f16kv_static(qd.data_ptr(), kc.data_ptr(), vc.data_ptr(), got.data_ptr(),
                                                        pd.data_ptr(), heads, kv, hd, max_seq, scale, s))
        torch.cuda.synchronize()
        a = got.cpu().numpy()
        b = want.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (heads, max_seq)
        kbits = kc.view(torch.int16).cpu().numpy().view(np.uint16).reshape(kv, max_seq, hd)
        vbits = vc.view(torch.int16).cpu().numpy().view(np.uint16).reshape(kv, max_seq, hd)
        expect = orc.attention_f16kv(q, kbits, vbits, heads, kv, hd, max_seq, pos, scale)
        assert close(a, expect, 1e-3) == 0


def test_static_attention_refuses_shapes_past_the_array(mh, gpu):
    torch = gpu
    lib = mh.load()
    # 8 kv heads x 16 chunks x group 8 x (128 + 2) floats = 532,480 bytes > 512 KiB.
    heads, kv, hd, max_seq = 64, 8, 128, 4096
    q = torch.zeros(heads * hd, dtype=torch.float32, device="cuda")
    kc = torch.zeros(kv * max_seq * hd, dtype=torch.float16, device="cuda")
    pd = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    status = lib.muyo_attention_decode_f16kv_static(q.data_ptr(), kc.data_ptr(), kc.data_ptr(), out.data_ptr(),
                                                     pd.data_ptr(), heads, kv, hd, max_seq, 0.1,
                                                     torch.cuda.current_stream().cuda_stream)
    assert status == mh.MUYO_E_UNSUPPORTED
    assert lib.muyo_attention_decode_f16kv_static(None, kc.data_ptr(), kc.data_ptr(), out.data_ptr(), pd.data_ptr(),
                                                  14, 2, 64, 256, 0.1, 0) == mh.MUYO_E_NULL
