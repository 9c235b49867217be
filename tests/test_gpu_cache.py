"""GPU: the activation cache with on-the-fly SAE encoding (reference tests/test_cache.py:91-99)
and the copy-stream path of a model that runs on the GPU."""

import numpy as np
import pytest
import torch

import saeflow_amd
from cache_model import BudgetedModel, ForwardBudgetExceeded, TinyHooked, hook_rows
from oracle import csr as ocsr
from oracle import reference as oref
from saeflow_amd.cache import ActivationReader, cache_activations
from saeflow_amd.kernels import csr_to_dense

pytestmark = pytest.mark.gpu

HOOKS = ["blocks.0.hook_resid_post", "blocks.1.attn.hook_z"]


@pytest.fixture
def tokens():
    return torch.randint(0, 100, (22, 16), generator=torch.Generator().manual_seed(1))


def collect(reader, hook, batch_size):
    """Every cached row of `hook`, read back in batches of `batch_size`."""
    return torch.cat([b for b in reader.iter_batches(hook, batch_size)])


def jumprelu_sae(d_in=32, d_sae=96, dtype=torch.float32):
    torch.manual_seed(0)
    sae = saeflow_amd.SAE(d_in, d_sae, "jumprelu", dtype=dtype, device="cuda")
    sae.threshold.fill_(0.5)
    return sae


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gpu_model_dense_hooks_read_back_exactly(tokens, tmp_path, dtype):
    model = TinyHooked(device="cuda").eval()
    cache_activations(model, tokens, HOOKS, tmp_path, batch_size=4, batches_per_shard=2, dtype=dtype)
    reader = ActivationReader(tmp_path)
    for hook in HOOKS:
        assert torch.equal(collect(reader, hook, 9), hook_rows(model, tokens, hook).to(dtype).cpu())


@pytest.mark.parametrize("model_device", ["cpu", "cuda"])
def test_encode_on_the_fly_stores_sparse(tokens, tmp_path, model_device):
    model = TinyHooked(device=model_device).eval()
    hook = HOOKS[0]
    sae = jumprelu_sae()
    cache_activations(model, tokens, [hook], tmp_path, batch_size=4, batches_per_shard=2, encoders={hook: sae})
    reader = ActivationReader(tmp_path)
    assert reader.manifest["hooks"][hook] == {"format": "csr", "d": 96}
    got = [tuple(t.cuda() for t in csr) for csr in reader.iter_batches(hook, 13)]
    dense = torch.cat([csr_to_dense(*csr, 96) for csr in got]).cpu()
    acts = hook_rows(model, tokens, hook).float()
    # the stored CSR is exactly what encode_sparse gives for the same activations
    want_csr = saeflow_amd.encode_sparse(sae, acts.cuda())
    assert torch.equal(dense, csr_to_dense(*want_csr, 96).cpu())
    # and matches the oracle (reference tolerance, test_cache.py:99)
    want = oref.encode(acts.cpu(), sae.W_enc, sae.b_enc, sae.b_dec, sae.threshold, "jumprelu")
    torch.testing.assert_close(dense, want, atol=1e-4, rtol=1e-4)


def test_encoded_cache_resumes_after_interruption(tokens, tmp_path):
    model = TinyHooked(device="cuda").eval()
    sae = jumprelu_sae(dtype=torch.bfloat16)
    enc = {HOOKS[0]: sae}
    with pytest.raises(ForwardBudgetExceeded):
        cache_activations(BudgetedModel(model, 3), tokens, HOOKS, tmp_path, batch_size=4, batches_per_shard=2,
                          dtype=torch.bfloat16, encoders=enc)
    assert len(ActivationReader(tmp_path).manifest["shards"]) == 1
    cache_activations(model, tokens, HOOKS, tmp_path, batch_size=4, batches_per_shard=2, dtype=torch.bfloat16,
                      encoders=enc)
    reader = ActivationReader(tmp_path)
    assert len(reader.manifest["shards"]) == 3 and not list(tmp_path.rglob("*.tmp"))
    indptr, indices, values = next(reader.iter_batches(HOOKS[0], 10 ** 6))
    acts = hook_rows(model, tokens, HOOKS[0]).to(torch.bfloat16)
    w_ip, w_ind, w_val = saeflow_amd.encode_sparse(sae, acts)
    assert torch.equal(indptr, w_ip.cpu()) and torch.equal(indices, w_ind.cpu())
    assert np.array_equal(ocsr.to_bits(values), ocsr.to_bits(w_val))
    assert torch.equal(collect(reader, HOOKS[1], 50), hook_rows(model, tokens, HOOKS[1]).bfloat16().cpu())
