"""GPU parity of the LM heads (the last and largest linears of both models):

* DeepSeek ``launch_lm_head`` (plugins/kernels/deepseek-v4-sm89/native/
  deepseek_endpoint.cu:94-115,484-497; validator deepseek_endpoint.cpp:57-66):
  x bf16 [rows, 4096] . W bf16 [129280, 4096]^T -> fp32 logits, error bits
  64 (non-finite operand) and 128 (non-finite logit);
* the Qwen3-0.6B head (nvidia_qwen3_int4_execution_driver.cpp:16-67): a
  bank of 1..32-row GemmPlans over the tied [151936, 1024] weight, fp32 out.

Weights are drawn on the device (1 GB for DeepSeek); the oracle
(po_lm_head, the reference kernel's reduction order) checks a stride of
vocabulary rows.  Tolerance: the fp32 sums run in a different order, so each
logit must lie within K * 2^-24 * sum|x w| of the oracle's (the standard
bound for two orderings of a K-term fp32 sum), plus max_rel <= 1e-2 and
cos >= 0.9999 over the checked block.
"""
import numpy as np
import pytest

import oracle
from tests.helpers import assert_close, to_host

pytestmark = pytest.mark.gpu

DS_VOCAB, DS_HIDDEN = 129280, 4096
QW_VOCAB, QW_HIDDEN = 151936, 1024
WORD_STRIDE = 61


@pytest.fixture(scope="module", autouse=True)
def eng():
    import torch

    from pih_amd.device import engine_stream

    with engine_stream() as s:
        yield s
        torch.cuda.synchronize()


def _device_weight(vocab, hidden, seed):
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w = torch.empty(vocab, hidden, dtype=torch.bfloat16, device="cuda")
    for r0 in range(0, vocab, 16384):  # bounded fp32 staging
        r1 = min(vocab, r0 + 16384)
        w[r0:r1] = (torch.randn(r1 - r0, hidden, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    return w


@pytest.fixture(scope="module")
def ds_weight(eng):
    import torch

    w = _device_weight(DS_VOCAB, DS_HIDDEN, 1234)
    words = np.arange(0, DS_VOCAB, WORD_STRIDE)
    w_sub = to_host(w[torch.from_numpy(words).cuda()])
    yield w, words, w_sub
    del w
    torch.cuda.empty_cache()


def _x(rows, hidden, seed):
    import torch

    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randn(rows, hidden, generator=g, device="cuda").to(torch.bfloat16)


def _check_logits(got, x_bits, w_sub_bits, what):
    ref, err = oracle.lm_head(x_bits, w_sub_bits)
    assert err == 0
    xf = oracle.bf16_bits_to_f32(x_bits).astype(np.float64)
    wf = oracle.bf16_bits_to_f32(w_sub_bits).astype(np.float64)
    bound = x_bits.shape[1] * 2.0 ** -24 * (np.abs(xf) @ np.abs(wf).T)
    assert (np.abs(got.astype(np.float64) - ref) <= bound).all(), what
    assert_close(got, ref, what)


@pytest.mark.parametrize("rows", [1, 2, 5, 64, 65, 200, 300])
def test_deepseek_lm_head(ds_weight, rows):
    """One row runs the weight-streaming GEMV; more (the vocabulary is more
    than a round of 256-column tiles) the persistent big tiles, one M tile
    up to 128 rows."""
    from pih_amd.linear import deepseek_lm_head

    w, words, w_sub = ds_weight
    x = _x(rows, DS_HIDDEN, 70 + rows)
    logits, flag = deepseek_lm_head(x, w)
    import torch

    torch.cuda.synchronize()
    assert int(flag.item()) == 0
    got = logits.cpu().numpy()[:, words]
    _check_logits(got, to_host(x), w_sub, f"deepseek lm_head rows={rows}")


@pytest.mark.parametrize("rows", [1, 2, 40, 100])
def test_deepseek_lm_head_error_bits(ds_weight, rows):
    import torch

    from pih_amd.linear import deepseek_lm_head

    w, words, _ = ds_weight
    x = _x(rows, DS_HIDDEN, 90 + rows)
    # a +inf weight element: that word's logits are non-finite, bits 64 | 128
    word = int(words[3])
    saved = w[word, 100].clone()
    w[word, 100] = float("inf")
    try:
        logits, flag = deepseek_lm_head(x, w)
        torch.cuda.synchronize()
        assert int(flag.item()) == 64 | 128
        got = logits.cpu().numpy()
        assert not np.isfinite(got[:, word]).any()
        assert np.isfinite(got[:, words[:3]]).all() and np.isfinite(got[:, words[4:]]).all()
    finally:
        w[word, 100] = saved
    # a NaN input element: that row's logits are NaN, bits 64 | 128
    x2 = x.clone()
    x2[rows - 1, 7] = float("nan")
    logits, flag = deepseek_lm_head(x2, w)
    torch.cuda.synchronize()
    assert int(flag.item()) == 64 | 128
    assert np.isnan(logits[rows - 1].cpu().numpy()).all()
    # finite operands whose products overflow fp32 (x row 0 and W row `word`
    # all 2^100): that one logit is non-finite, bit 128 only
    saved_row = w[word].clone()
    w[word] = 2.0 ** 100
    try:
        x3 = x.clone()
        x3[0] = 2.0 ** 100
        logits, flag = deepseek_lm_head(x3, w)
        torch.cuda.synchronize()
        assert int(flag.item()) == 128
        got = logits.cpu().numpy()
        assert not np.isfinite(got[0, word]) and np.isfinite(got[1:, word]).all()
    finally:
        w[word] = saved_row


def test_deepseek_lm_head_validation(ds_weight):
    import torch

    from pih_amd import abi
    from pih_amd.device import ptr, stream_handle

    w, _, _ = ds_weight
    x = _x(4, DS_HIDDEN, 5)
    out = torch.empty(4, DS_VOCAB, dtype=torch.float32, device="cuda")
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    base = dict(input_bf16=ptr(x), weight_bf16=ptr(w), logits_f32=ptr(out), error_flag_u32=ptr(flag),
                stream=stream_handle(), output_rows=4, vocab_size=DS_VOCAB, hidden_size=DS_HIDDEN)
    pack = abi.deepseek_pack()
    assert pack.call("launch_lm_head", abi.request(abi.DS["lm_head"], **base)).code == abi.OK
    for bad in (dict(vocab_size=129279), dict(hidden_size=4095), dict(output_rows=0), dict(output_rows=4097),
                dict(logits_f32=ptr(x)), dict(error_flag_u32=0), dict(stream=0)):
        st = pack.call("launch_lm_head", abi.request(abi.DS["lm_head"], **{**base, **bad}))
        assert st.code == abi.INVALID_ARGUMENT, bad
    torch.cuda.synchronize()


@pytest.fixture(scope="module")
def qw_weight(eng):
    import torch

    w = _device_weight(QW_VOCAB, QW_HIDDEN, 4321)
    words = np.arange(0, QW_VOCAB, WORD_STRIDE)
    yield w, words, to_host(w[torch.from_numpy(words).cuda()])
    del w
    torch.cuda.empty_cache()


@pytest.mark.parametrize("rows", [1, 7, 32])
def test_qwen_lm_head_plan_bank(qw_weight, rows):
    import torch

    from pih_amd.linear import QwenLmHead

    w, words, w_sub = qw_weight
    head = QwenLmHead(32)
    x = _x(rows, QW_HIDDEN, 200 + rows)
    out = torch.empty(rows, QW_VOCAB, dtype=torch.float32, device="cuda")
    head.execute(x, w, out)
    torch.cuda.synchronize()
    _check_logits(out.cpu().numpy()[:, words], to_host(x), w_sub, f"qwen lm head rows={rows}")


def test_qwen_lm_head_bank_limits(qw_weight):
    import torch

    from pih_amd.linear import QwenLmHead

    w, _, _ = qw_weight
    for bad in (0, 33):
        with pytest.raises(ValueError):
            QwenLmHead(bad)
    head = QwenLmHead(4)
    x = _x(5, QW_HIDDEN, 9)
    out = torch.empty(5, QW_VOCAB, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError):
        head.execute(x, w, out)
