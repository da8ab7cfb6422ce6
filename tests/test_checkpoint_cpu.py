"""Checkpoint loading without a GPU: 8-bit AdamW states keep their uint8 codes and
fp32 block scales / codebooks through load_state_dict (format_version 2,
muon_sr/triton_adamw_8bit.py:207-241), in TritonAdamW8bit and in the hybrid
optimizer's optim_bits=8 AdamW groups (torch's default load would cast every
state tensor to the bf16 parameter dtype)."""
import pytest
import torch

from muon_sr_amd import TritonAdamW8bit, TritonMuonSRWithAuxAdam


def state_8bit(shape, block=256):
    n = 1
    for s in shape:
        n *= s
    nb = -(-n // block)
    return dict(step=3, format_version=2, block_size=block, optim_bits=8,
                state1=torch.full(shape, 127, dtype=torch.uint8), state2=torch.arange(n, dtype=torch.uint8).reshape(shape),
                qmap1=torch.linspace(-1, 1, 256), qmap2=torch.linspace(0, 1, 256),
                absmax1=torch.full((nb,), 1.2345678), absmax2=torch.full((nb,), 3e-9))


@pytest.mark.parametrize("which", ["8bit", "hybrid"])
def test_load_keeps_8bit_dtypes(which):
    p = torch.nn.Parameter(torch.zeros(64, 96, dtype=torch.bfloat16))
    q = torch.nn.Parameter(torch.zeros(40, dtype=torch.bfloat16))
    if which == "8bit":
        opt = TritonAdamW8bit([p, q], lr=1e-3)
    else:
        opt = TritonMuonSRWithAuxAdam([dict(params=[p, q], use_muon=False, optim_bits=8)])
    sd = opt.state_dict()
    saved = state_8bit((64, 96))
    small = dict(step=3, format_version=2, block_size=256, optim_bits=16,
                 state1=torch.full((40,), 0.25, dtype=torch.bfloat16), state2=torch.zeros(40, dtype=torch.bfloat16))
    sd["state"] = {0: saved, 1: small}
    opt.load_state_dict(sd)
    st = opt.state[p]
    for k in ("state1", "state2"):
        assert st[k].dtype == torch.uint8 and torch.equal(st[k], saved[k])
    for k in ("qmap1", "qmap2", "absmax1", "absmax2"):
        assert st[k].dtype == torch.float32 and torch.equal(st[k], saved[k])
    assert st["step"] == 3 and st["format_version"] == 2
    assert opt.state[q]["state1"].dtype == torch.bfloat16 and torch.equal(opt.state[q]["state1"], small["state1"])
    # the loaded tensors are copies, not the checkpoint's storage
    assert st["absmax1"].data_ptr() != saved["absmax1"].data_ptr()


def test_hybrid_rejects_incompatible_8bit_state():
    p = torch.nn.Parameter(torch.zeros(64, 96, dtype=torch.bfloat16))
    opt = TritonMuonSRWithAuxAdam([dict(params=[p], use_muon=False, optim_bits=8)])
    sd = opt.state_dict()
    bad = state_8bit((64, 96))
    bad["absmax1"] = bad["absmax1"].to(torch.bfloat16)
    sd["state"] = {0: bad}
    with pytest.raises(ValueError, match="Invalid checkpoint state: absmax1"):
        opt.load_state_dict(sd)
    bad = state_8bit((64, 96), block=128)
    sd["state"] = {0: bad}
    with pytest.raises(ValueError, match="Incompatible state format"):
        opt.load_state_dict(sd)



def _reference_checkpoints():
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "checkpoints.pt")
    return torch.load(path, weights_only=True)


@pytest.mark.parametrize("case", ["adamw", "adamw8bit", "muon_batch", "hybrid_batch"])
def test_reference_checkpoint_loads_and_saves_unchanged(case):
    """A state_dict the reference's own class wrote (tests/golden/checkpoints.pt) loads into
    this library's class and comes back out of state_dict() unchanged: same param groups,
    state keys, dtypes, shapes and values (muon_sr/triton_adamw_8bit.py:207-241,
    muon_sr/muon_sr.py:149-158)."""
    from muon_sr_amd import TritonAdamW, TritonMuonSR
    rec = _reference_checkpoints()[case]
    ps = [torch.nn.Parameter(p.clone()) for p in rec["p_ckpt"]]
    if case == "adamw":
        opt = TritonAdamW([{"params": ps[:2]}, {"params": ps[2:], "lr": 2e-3, "weight_decay": 0.1,
                                                 "centralization": 0.5}], lr=1e-3, betas=(0.9, 0.95), eps=1e-8)
    elif case == "adamw8bit":
        opt = TritonAdamW8bit([{"params": ps[:2]}, {"params": ps[2:], "optim_bits": 16}],
                              lr=3e-4, betas=(0.9, 0.95), eps=1e-10, weight_decay=0.01)
    elif case == "muon_batch":
        opt = TritonMuonSR(ps, lr=0.02, weight_decay=0.01, batch_ns=True)
    else:
        opt = TritonMuonSRWithAuxAdam(
            [{"params": ps[:3], "use_muon": True, "weight_decay": 0.01},
             {"params": ps[3:], "use_muon": False, "lr": 3e-4, "betas": (0.9, 0.95), "eps": 1e-10,
              "weight_decay": 0.01}], batch_ns=True)
    ref = rec["state_dict"]
    opt.load_state_dict(ref)
    out = opt.state_dict()
    assert out["param_groups"] == ref["param_groups"]
    assert sorted(out["state"]) == sorted(ref["state"])
    for i, st in ref["state"].items():
        assert sorted(out["state"][i]) == sorted(st), i
        for k, v in st.items():
            w = out["state"][i][k]
            if torch.is_tensor(v):
                assert w.dtype == v.dtype and w.shape == v.shape and torch.equal(w.view(-1).view(torch.uint8) if w.dtype == torch.bfloat16 else w,
                                                                                  v.view(-1).view(torch.uint8) if v.dtype == torch.bfloat16 else v), (i, k)
            else:
                assert w == v, (i, k)
