"""qlin_moe_routed_decode_grouped_noalloc (no counterpart in the reference): the batched routed MoE decode
on the library's per-GPU scratch array, for callers that cannot allocate.  It must give exactly what
qlin_moe_routed_decode_grouped gives with a workspace of the caller's: the same kernels on the same
inputs, bit for bit, on two calls in a row (the second with fewer tokens, on the contents the first
left in the shared array), and it must refuse a batch beyond the array's size before anything runs."""
import numpy as np
import pytest
import torch

import oracle as orc
import qgen
from blog_amd import qlin
from gpu_util import banner, bind_stream, dev, host
from qgen import Q4_K, Q5_0, Q6_K

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _stream():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    bind_stream()
    yield
    torch.cuda.synchronize()


E, FFN, HID, K = 16, 512, 1024, 4


def _experts(gu_type, e, ffn, hid, seed):
    wg, _, _ = qgen.random_matrix(gu_type, e * ffn, hid, seed=seed)
    wu, _, _ = qgen.random_matrix(gu_type, e * ffn, hid, seed=seed + 1)
    wd, _, _ = qgen.random_matrix(Q5_0, e * hid, ffn, seed=seed + 2)
    return dev(wg), dev(wu), dev(wd), wg.size, wd.size


@pytest.fixture(scope="module")
def experts():
    return _experts(Q4_K, E, FFN, HID, 1201)


def _inputs(tokens, e, hid, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((tokens, hid)).astype(np.float32)
    ids, rw = orc.router_topk(rng.standard_normal((tokens, e)).astype(np.float32), K, 1.0)
    ids = np.ascontiguousarray(ids)
    ids[0, 1] = -1  # a route without an expert
    out0 = rng.standard_normal((tokens, hid)).astype(np.float32)
    return x, ids, np.ascontiguousarray(rw), out0


# Every path that runs on the shared scratch, each on two calls in a row with fewer tokens the second
# time (the second call reads the array the first one left): the gate/up launch grouping the routes
# itself (16 experts, 48 and 12 routes); group_kernel first, for more than 256 experts and for more
# than 1024 routes; and the per-token kernels with act in the scratch (Q6_K gate/up, which the grouped
# kernels do not take).
CASES = [("in-kernel grouping", Q4_K, E, FFN, HID, (12, 3)),
         ("group_kernel: 300 experts", Q4_K, 300, 64, 256, (12, 3)),
         ("group_kernel: 1200 routes", Q4_K, 16, 64, 256, (300, 260)),
         ("per-token Q6_K gate/up", Q6_K, 16, 128, 512, (6, 2))]


@pytest.mark.parametrize("name,gu_type,e,ffn,hid,calls", CASES, ids=[c[0] for c in CASES])
def test_noalloc_equals_workspace_entry_on_two_calls(name, gu_type, e, ffn, hid, calls):
    wg, wu, wd, gub, db = _experts(gu_type, e, ffn, hid, 1201 + e + ffn)
    for call, tokens in enumerate(calls):
        x, ids, rw, out0 = _inputs(tokens, e, hid, 1210 + call + e)
        xd, idd, rwd = dev(x), dev(ids), dev(rw)
        banner(f"moe noalloc {name} call {call} tokens={tokens}")
        nbytes = qlin.lib().qlin_moe_grouped_workspace_bytes(tokens, K, e, ffn, hid)
        assert nbytes <= (8 << 20)
        ws = torch.empty(nbytes + 256, dtype=torch.uint8, device="cuda")
        wsp = (ws.data_ptr() + 255) // 256 * 256
        out_ws = dev(out0)
        qlin.call("qlin_moe_routed_decode_grouped", gu_type, wg, wu, gub, Q5_0, wd, db, e, ffn, hid, hid, xd, idd,
                  rwd, wsp, nbytes, out_ws, tokens, K)
        out_na = dev(out0)
        qlin.call("qlin_moe_routed_decode_grouped_noalloc", gu_type, wg, wu, gub, Q5_0, wd, db, e, ffn, hid, hid, xd,
                  idd, rwd, out_na, tokens, K)
        a, b = host(out_na), host(out_ws)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert not np.array_equal(a, out0)


def test_noalloc_refuses_a_batch_beyond_its_scratch(experts):
    wg, wu, wd, gub, db = experts
    tokens = 1024  # 4096 routes x (512 + 1024) floats: 25 MB of workspace
    assert qlin.lib().qlin_moe_grouped_workspace_bytes(tokens, K, E, FFN, HID) > (8 << 20)
    x = torch.zeros(tokens, HID, device="cuda")
    ids = torch.zeros(tokens, K, dtype=torch.int32, device="cuda")
    rw = torch.ones(tokens, K, device="cuda")
    out = torch.full((tokens, HID), 3.0, device="cuda")
    rc = qlin.lib().qlin_moe_routed_decode_grouped_noalloc(Q4_K, wg.data_ptr(), wu.data_ptr(), gub, Q5_0,
                                                          wd.data_ptr(), db, E, FFN, HID, HID, x.data_ptr(),
                                                          ids.data_ptr(), rw.data_ptr(), out.data_ptr(), tokens, K)
    assert qlin.STATUS[rc] == "QLIN_ERR_LIMIT"
    assert torch.all(out == 3.0)
