"""The int8 LM head at vocabulary width (row a14): `LMHead(QTensor)` over
Qwen3-8B's [151936, 4096] head, fed the strided last-position slice
`hidden[:, -1]` (row stride S*hidden; fni8serve/layers/embedding.py:49-53).

Bars: sampled vocabulary columns bit for bit against the oracle, and the
reference's own check of a quantized head (tests/test_lm_head_quant.py:45-53):
cosine > 0.999 against the fp16 head and the same argmax on every row."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle

pytestmark = pytest.mark.gpu

VOCAB, HIDDEN = 151936, 4096


@pytest.fixture(scope="module")
def head(pkg, cuda):
    g = torch.Generator().manual_seed(31)
    w = (torch.randn(VOCAB, HIDDEN, generator=g) * 0.02).half()   # the fp16 head (tied embedding)
    wd = w.to(cuda)
    q, s = pkg.quantize_int8_rowwise(wd)                            # to_qtensor's weight quantization
    qt = pkg.QTensor(q, s.reshape(-1).float().contiguous(), scheme="per_row_i8")
    return pkg.LMHead(qt), wd, qt


@pytest.mark.parametrize("B", [1, 4, 32])
def test_lm_head_vocab_width(pkg, cuda, head, B):
    lm, wd, qt = head
    hidden = torch.randn(B, 3, HIDDEN, generator=torch.Generator().manual_seed(40 + B)).half()
    last = hidden.to(cuda)[:, -1]
    assert last.stride(0) == 3 * HIDDEN and (B == 1 or not last.is_contiguous())
    logits = lm(last)
    torch.cuda.synchronize()
    assert logits.shape == (B, VOCAB) and logits.dtype == torch.float16
    # sampled vocabulary columns, bit for bit
    rng = np.random.default_rng(B)
    ref = F.linear(last.float(), wd.float())                  # the fp16 head, in fp32
    cols = np.unique(np.concatenate([[0, VOCAB - 1], rng.choice(VOCAB, 500, replace=False),
                                     ref.argmax(-1).cpu().numpy()]))
    q = qt.data.cpu().numpy()[cols]
    s = qt.scale.cpu().numpy()[cols]
    yr, _, _, _ = oracle.linear_w8a8_f16(hidden[:, -1].contiguous().numpy(), q, s, None)
    got = logits.cpu().numpy()[:, cols]
    assert np.array_equal(got.view(np.uint16), yr.view(np.uint16))
    # the reference's bar for a quantized head
    cos = F.cosine_similarity(logits.float(), ref, dim=-1)
    assert cos.min().item() > 0.999, f"cosine {cos.min().item():.5f}"
    assert torch.equal(logits.float().argmax(-1), ref.argmax(-1))
