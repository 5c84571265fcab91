"""CPU checks of the config-5 harness (tests/minigpt.py): the model has the
BASELINE dimensions, the reference-restatement build starts from the same
weights as the fp32 model, and one training step of it runs on the CPU."""
from __future__ import annotations

import torch

import minigpt


def test_config5_dimensions():
    c = minigpt.GPTConfig()
    assert (c.num_layers, c.embed_dim, c.num_heads, c.ff_dim, c.vocab_size, c.context_len, c.batch) == \
        (4, 256, 4, 1024, 256, 128, 64)
    m = minigpt.base_model(0)
    n_linear = sum(isinstance(t, torch.nn.Linear) for t in m.modules())
    assert n_linear == 4 * 6 + 1
    x, y = minigpt.batch(1)
    assert x.shape == (64, 128) and y.shape == (64, 128) and torch.equal(x[:, 1:], y[:, :-1])


def test_reference_build_shares_initial_weights():
    fp32 = minigpt.base_model(0)
    ref = minigpt.build_reference(0)
    p1 = dict(fp32.named_parameters())
    p2 = dict(ref.named_parameters())
    assert p1.keys() == p2.keys()
    for k in p1:
        assert torch.equal(p1[k], p2[k]), k


def test_reference_step_runs_and_tracks_fp32():
    torch.set_num_threads(max(1, min(8, torch.get_num_threads())))
    x, y = minigpt.batch(1)
    x, y = x[:8], y[:8]
    ref_losses, _ = minigpt.train(minigpt.build_reference(0), x, y, 2)
    fp_losses, _ = minigpt.train(minigpt.base_model(0), x, y, 2)
    # NF5 fake quantization of weights and activations moves the initial loss
    # only slightly (the network is near-uniform at init)
    assert abs(ref_losses[0] - fp_losses[0]) / fp_losses[0] < 1e-3
    assert ref_losses[1] < ref_losses[0]
