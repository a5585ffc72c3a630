"""Forwards replayed as HIP graphs (eii_model_set_graphs) equal the eagerly launched forward: several
replays of one captured graph with other eager work and synchronizations between them, a second shape
captured beside the first, and the plain launches again after graphs are switched off."""
import ctypes as C

import numpy as np
import pytest
import torch

from eii import lib as L
from eii import synth

pytestmark = pytest.mark.gpu


def _forward(eng, ids, logits, emb, res, B, T):
    L.check(eng.lib.eii_forward(eng.h, C.c_void_p(ids.data_ptr()), B, T, C.c_void_p(emb.data_ptr()),
                                C.c_void_p(res.data_ptr()), C.c_void_p(logits.data_ptr()), None,
                                C.c_void_p(torch.cuda.current_stream().cuda_stream)))


def test_graph_replays_match_eager(model_path):
    from eii.engine import Engine
    eng = Engine(model_path)
    try:
        ids_a = torch.from_numpy(synth.token_ids("cfg1")).cuda()                  # 1 x 24
        ids_b = torch.from_numpy(synth.token_ids("cfg4")[:3, :40].copy()).cuda()   # 3 x 40
        want_a = eng.forward(ids_a, embed=True, resid=True, logits=True)
        want_b = eng.forward(ids_b, embed=True, resid=True, logits=True)
        eng.set_graphs(True)
        bufs = {}
        for name, ids in (("a", ids_a), ("b", ids_b)):
            B, T = ids.shape
            bufs[name] = (ids, torch.empty((B * T, 49152), dtype=torch.int32, device="cuda"),
                          torch.empty((B * T, 576), dtype=torch.int32, device="cuda"),
                          torch.empty((30, B * T, 576), dtype=torch.int32, device="cuda"), B, T)
        for rep in range(4):
            for name, want in (("a", want_a), ("b", want_b)):
                ids, lg, emb, res, B, T = bufs[name]
                for t in (lg, emb, res):
                    t.fill_(-7)                          # stale values must be overwritten by each replay
                _forward(eng, ids, lg, emb, res, B, T)
                torch.cuda.synchronize()
                eng.check()
                assert torch.equal(lg.view(B, T, -1), want["logits"]), (name, rep)
                assert torch.equal(emb.view(B, T, -1), want["embed"]), (name, rep)
                assert torch.equal(res.view(30, B, T, -1), want["resid"]), (name, rep)
            # eager work between the replays
            x = torch.arange(1 << 20, device="cuda", dtype=torch.int64).sum()
            assert int(x) == (1 << 20) * ((1 << 20) - 1) // 2
        eng.set_graphs(False)
        again = eng.forward(ids_a, embed=True, resid=True, logits=True)
        for k in ("logits", "embed", "resid"):
            assert torch.equal(again[k], want_a[k]), k
    finally:
        eng.close()
