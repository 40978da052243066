"""The no-allocation pair scan (tq_ip_scan_topk_pairs_noalloc, static per-GPU scratch)
against tq_ip_scan_topk_pairs with a caller workspace, through the C ABI: two calls in a
row, the second smaller, must return the same scores and ids bit for bit; a request
beyond the static scratch is refused before any launch."""

import ctypes

import numpy as np
import pytest
import torch

import capi

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def L():
    lib = capi.lib()
    lib.tq_ip_scan_topk_pairs_noalloc.restype = ctypes.c_int
    return lib


def _db(rs, N, d):
    pairs = torch.from_numpy(rs.randint(0, 256, (N, d // 2)).astype(np.uint8)).to(DEV)
    norms = torch.from_numpy(rs.uniform(0.5, 2.0, N).astype(np.float32)).to(DEV)
    return pairs, norms


def _tables(rs, d):
    R = torch.from_numpy(np.linalg.qr(rs.randn(d, d))[0].astype(np.float32)).to(DEV)
    cen = torch.from_numpy(np.sort(rs.randn(16)).astype(np.float32) / np.sqrt(d)).to(DEV)
    return R, cen


def _with_workspace(q, pairs, norms, cen, R, k):
    nq, d = q.shape
    N = pairs.shape[0]
    s = torch.empty(nq, k, dtype=torch.float32, device=DEV)
    i = torch.empty(nq, k, dtype=torch.int64, device=DEV)
    ws = torch.empty(L().tq_scan_workspace_bytes(nq, d, 4, N, k), dtype=torch.uint8, device=DEV)
    capi.check(L().tq_ip_scan_topk_pairs(capi.p(q), capi.TQ_F16, capi.i64(nq), capi.i32(d),
                                         capi.p(pairs), capi.p(norms), capi.i64(N), capi.p(cen),
                                         capi.p(R), capi.i32(k), capi.p(s), capi.p(i), capi.p(ws),
                                         ctypes.c_size_t(ws.numel()), capi.stream()))
    return s, i


def _noalloc(q, pairs, norms, cen, R, k):
    nq, d = q.shape
    N = pairs.shape[0]
    s = torch.empty(nq, k, dtype=torch.float32, device=DEV)
    i = torch.empty(nq, k, dtype=torch.int64, device=DEV)
    rc = L().tq_ip_scan_topk_pairs_noalloc(capi.p(q), capi.TQ_F16, capi.i64(nq), capi.i32(d),
                                           capi.p(pairs), capi.p(norms), capi.i64(N), capi.p(cen),
                                           capi.p(R), capi.i32(k), capi.p(s), capi.p(i),
                                           capi.stream())
    return rc, s, i


@pytest.mark.parametrize("d", [128, 64])
def test_noalloc_scan_equals_workspace_scan(d):
    rs = np.random.RandomState(d)
    R, cen = _tables(rs, d)
    # first call: 3 queries over 300k rows, k = 10; second: 1 query over 50k rows, k = 7
    for nq, N, k in ((3, 300_000, 10), (1, 50_000, 7)):
        print(f"noalloc scan d={d} nq={nq} N={N} k={k}", flush=True)
        pairs, norms = _db(rs, N, d)
        q = torch.from_numpy(rs.randn(nq, d).astype(np.float32)).to(DEV).half()
        rc, s, i = _noalloc(q, pairs, norms, cen, R, k)
        capi.check(rc)
        ws_s, ws_i = _with_workspace(q, pairs, norms, cen, R, k)
        torch.cuda.synchronize()
        assert torch.equal(i, ws_i)
        assert torch.equal(s.view(torch.int32), ws_s.view(torch.int32))


def test_noalloc_scan_rejects_requests_beyond_its_scratch():
    rs = np.random.RandomState(3)
    d, N, k = 128, 2_000_000, 32
    limit = L().tq_scan_workspace_bytes(1, d, 4, N, k)
    nq = 2
    while L().tq_scan_workspace_bytes(nq, d, 4, N, k) <= (4 << 20):
        nq *= 2
    R, cen = _tables(rs, d)
    pairs = torch.zeros(N, d // 2, dtype=torch.uint8, device=DEV)
    norms = torch.ones(N, dtype=torch.float32, device=DEV)
    q = torch.zeros(nq, d, dtype=torch.float16, device=DEV)
    rc, _, _ = _noalloc(q, pairs, norms, cen, R, k)
    assert rc == 1 and b"static" in L().tq_last_error()
    assert limit <= (4 << 20)
