"""GPU parity of the elementwise / attention operators against the oracle."""
import numpy as np
import pytest

import oracle as O
from tests.helpers import rel_err

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("n", [4, 768, 2048, 5000])
def test_rmsnorm_layernorm(gpu, n):
    from smallmind_amd.quantization import layernorm, rmsnorm
    rng = np.random.default_rng(n)
    x = rng.normal(0, 2, (3, n)).astype(np.float32)
    g = rng.normal(1, 0.2, n).astype(np.float32)
    b = rng.normal(0, 0.2, n).astype(np.float32)
    assert rel_err(rmsnorm(_dev(x), _dev(g)).cpu().numpy(), O.rmsnorm(x, g)) < 2e-6
    assert rel_err(layernorm(_dev(x), _dev(g), _dev(b)).cpu().numpy(), O.layernorm(x, g, b)) < 2e-6


def test_rmsnorm_reference_values(gpu):
    from smallmind_amd.quantization import rmsnorm
    x = np.array([[0.5, 1.5, 2.5, 3.5]], np.float32)
    g = np.array([1.2, 0.8, 1.5, 0.5], np.float32)
    inv = 1.0 / np.sqrt((0.25 + 2.25 + 6.25 + 12.25) / 4 + 1e-5)
    assert np.allclose(rmsnorm(_dev(x), _dev(g)).cpu().numpy(), g * x * inv, atol=1e-4)


def test_rope_tables_equal_oracle_and_apply(gpu):
    from smallmind_amd.quantization import rope_, rope_tables
    c, s = rope_tables(300, 64, 10000.0)
    oc, os_ = O.rope_tables(300, 64, 10000.0)
    assert np.array_equal(c, oc) and np.array_equal(s, os_)
    rng = np.random.default_rng(0)
    x = rng.normal(0, 1, (4, 6, 64)).astype(np.float32)
    got = rope_(_dev(x), 37, _dev(c), _dev(s)).cpu().numpy()
    assert np.array_equal(got, O.rope_apply(x, 37, oc, os_))
    got0 = rope_(_dev(x), 0, _dev(c), _dev(s)).cpu().numpy()
    assert np.array_equal(got0[:, 0], x[:, 0])   # position 0 is the identity


@pytest.mark.parametrize("seq,kseq,off", [(1, 1, 0), (1, 700, 699), (5, 9, 4), (3, 3000, 2997)])
def test_scale_mask_softmax(gpu, seq, kseq, off):
    from smallmind_amd.quantization import scale_mask_softmax_
    s = np.random.default_rng(kseq).normal(0, 3, (seq, kseq)).astype(np.float32)
    got = scale_mask_softmax_(_dev(s), 0.125, off).cpu().numpy()
    ref = O.scale_mask_softmax(s, 0.125, off)
    assert np.abs(got - ref).max() < 1e-6
    for i in range(seq):
        assert np.all(got[i, off + i + 1:] == 0)


@pytest.mark.parametrize("H,Hkv,hd,npos", [(32, 4, 64, 1), (32, 4, 64, 513), (12, 12, 64, 160),
                                           (32, 32, 64, 300), (8, 2, 128, 1000), (32, 4, 64, 4096),
                                           (12, 4, 32, 33), (16, 1, 16, 95), (4, 4, 128, 31),
                                           (16, 2, 64, 767), (32, 4, 64, 1500), (8, 8, 64, 2500),
                                           (32, 4, 64, 4608), (4, 2, 64, 5000)])
def test_attention_decode_vs_oracle(gpu, H, Hkv, hd, npos):
    from smallmind_amd.quantization import attention_decode
    rng = np.random.default_rng(npos)
    ctx = npos + 7
    q = rng.normal(0, 1, (H, hd)).astype(np.float32)
    kc = rng.normal(0, 1, (Hkv, ctx, hd)).astype(np.float32)
    vc = rng.normal(0, 1, (Hkv, ctx, hd)).astype(np.float32)
    kt = np.ascontiguousarray(kc.transpose(0, 2, 1))   # the backend keeps K dimension-major
    got = attention_decode(_dev(q), _dev(kt), _dev(vc), H, Hkv, hd, ctx, npos).cpu().numpy()
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    ref = np.empty((H, hd), np.float32)
    for h in range(H):
        kv = h // (H // Hkv)
        sc = (kc[kv, :npos].astype(np.float64) @ q[h].astype(np.float64)).astype(np.float32)[None]
        p = O.scale_mask_softmax(sc, float(scale), cache_off=npos - 1)[0]
        ref[h] = p.astype(np.float64) @ vc[kv, :npos].astype(np.float64)
    assert rel_err(got.reshape(H, hd), ref) < 1e-5


@pytest.mark.parametrize("H,Hkv,hd,npos,ctx", [(32, 4, 64, 1, 4), (32, 4, 64, 160, 160), (12, 12, 64, 255, 256),
                                               (32, 4, 64, 256, 260), (8, 2, 64, 257, 512), (32, 4, 64, 511, 512),
                                               (32, 4, 64, 700, 768), (32, 4, 64, 768, 768), (16, 4, 64, 769, 1024),
                                               (32, 8, 64, 1024, 1024), (12, 4, 32, 600, 604), (16, 1, 16, 95, 100),
                                               (4, 4, 32, 1000, 1000)])
def test_attention_decode_one_launch_vs_oracle(gpu, H, Hkv, hd, npos, ctx):
    """Contexts up to 1024 positions with 16-byte aligned cache rows (ctx % 4 == 0) run as one
    launch that computes the scores inside the P.V workgroups.  Cache entries past n_pos hold
    NaN: they must never reach the output."""
    from smallmind_amd.quantization import attention_decode
    rng = np.random.default_rng(npos * 3 + hd)
    q = rng.normal(0, 1, (H, hd)).astype(np.float32)
    kc = rng.normal(0, 1, (Hkv, ctx, hd)).astype(np.float32)
    vc = rng.normal(0, 1, (Hkv, ctx, hd)).astype(np.float32)
    kc[:, npos:] = np.nan
    vc[:, npos:] = np.nan
    kt = np.ascontiguousarray(kc.transpose(0, 2, 1))
    got = attention_decode(_dev(q), _dev(kt), _dev(vc), H, Hkv, hd, ctx, npos).cpu().numpy().reshape(H, hd)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    ref = np.empty((H, hd), np.float32)
    for h in range(H):
        kv = h // (H // Hkv)
        sc = (kc[kv, :npos].astype(np.float64) @ q[h].astype(np.float64)).astype(np.float32)[None]
        p = O.scale_mask_softmax(sc, float(scale), cache_off=npos - 1)[0]
        ref[h] = p.astype(np.float64) @ vc[kv, :npos].astype(np.float64)
    assert np.isfinite(got).all()
    assert rel_err(got, ref) < 1e-5


@pytest.mark.parametrize("H,Hkv,p0,n", [(32, 4, 0, 37), (32, 4, 300, 64), (12, 12, 5, 33),
                                        (16, 1, 0, 20), (8, 8, 1000, 17), (4, 2, 0, 1),
                                        (32, 32, 255, 256), (32, 4, 3840, 256), (2, 2, 16, 48)])
def test_attention_prefill_vs_oracle(gpu, H, Hkv, p0, n):
    """Causal attention of n tokens at positions p0.. over the cache (MultiHeadAttention T > 1).
    Cache entries past the last token hold NaN: they must never reach the output."""
    from smallmind_amd.quantization import attention_prefill
    hd = 64
    rng = np.random.default_rng(p0 * 7 + n)
    ctx = p0 + n + 9
    q = rng.normal(0, 1, (n, H, hd)).astype(np.float32)
    kc = rng.normal(0, 1, (Hkv, ctx, hd)).astype(np.float32)
    vc = rng.normal(0, 1, (Hkv, ctx, hd)).astype(np.float32)
    kc[:, p0 + n:] = np.nan
    vc[:, p0 + n:] = np.nan
    kt = np.ascontiguousarray(kc.transpose(0, 2, 1))   # the backend keeps K dimension-major
    got = attention_prefill(_dev(q), _dev(kt), _dev(vc), H, Hkv, hd, ctx, p0, n).cpu().numpy()
    got = got.reshape(n, H, hd)
    scale = np.float32(1.0) / np.sqrt(np.float32(hd))
    ref = np.empty((n, H, hd), np.float32)
    kl = p0 + n
    for h in range(H):
        kv = h // (H // Hkv)
        sc = (q[:, h].astype(np.float64) @ kc[kv, :kl].astype(np.float64).T).astype(np.float32)
        p = O.scale_mask_softmax(sc, float(scale), cache_off=p0)
        ref[:, h] = p.astype(np.float64) @ vc[kv, :kl].astype(np.float64)
    assert np.isfinite(got).all()
    assert rel_err(got, ref) < 2e-5


def test_silu_mul_gelu(gpu):
    from smallmind_amd.quantization import gelu, silu_mul
    rng = np.random.default_rng(1)
    g = rng.normal(0, 4, 10001).astype(np.float32)
    u = rng.normal(0, 1, 10001).astype(np.float32)
    assert np.allclose(silu_mul(_dev(g), _dev(u)).cpu().numpy(), O.silu_mul(g, u), rtol=2e-6, atol=1e-7)
    x = rng.normal(0, 3, 10001).astype(np.float32)
    assert np.allclose(gelu(_dev(x)).cpu().numpy(), O.gelu(x), rtol=1e-6, atol=1e-7)


def test_argmax_lowest_index_on_ties(gpu):
    from smallmind_amd.quantization import argmax
    rng = np.random.default_rng(2)
    for n in (1, 63, 32000, 50257):
        v = rng.normal(0, 1, n).astype(np.float32)
        assert argmax(_dev(v)) == int(np.argmax(v))
        if n > 10:
            v[n // 3] = v[n - 2] = v.max() + 1
            assert argmax(_dev(v)) == n // 3


SAMPLING = [dict(), dict(temperature=0.8, top_k=40, top_p=0.95), dict(temperature=0.7, min_p=0.05),
            dict(top_k=1), dict(top_p=0.1), dict(temperature=1.3, top_p=0.5, min_p=0.01),
            dict(repetition_penalty=1.3, presence_penalty=0.4, frequency_penalty=0.2, top_k=100),
            dict(repetition_penalty=1.1, repetition_window=20, temperature=0.5)]


@pytest.mark.parametrize("n", [1000, 32000, 50257])
@pytest.mark.parametrize("opts", range(len(SAMPLING)))
def test_sample_vs_oracle(gpu, n, opts):
    """smx_sample against the oracle pipeline: the final distributions agree to the rounding of
    the normalising sums (the reference adds up to 50K probabilities one by one in fp32, about
    3e-5 relative at this size; the kernel sums in a tree), and the drawn ids are identical
    except where u falls within that rounding of a CDF step."""
    import torch
    from smallmind_amd.quantization import sample
    kw = SAMPLING[opts]
    rng = np.random.default_rng(n + opts)
    logits = rng.normal(0, 3, n).astype(np.float32)
    ctx = rng.integers(0, n, 300).astype(np.int32)
    ctx[-40:] = ctx[-60:-20]   # repeats inside the window
    okw = dict(kw)
    if "repetition_window" in okw:
        okw["window"] = okw.pop("repetition_window")
    for u in rng.random(6):
        tok, p = sample(_dev(logits), u, context=_dev(ctx), **kw)
        otok, op = O.sample(logits, u, context=ctx, **okw)
        p = p.cpu().numpy()
        # kept sets: equal unless the top-p cumulative sum sits within rounding of the cutoff
        if not np.array_equal(p > 0, op > 0):
            base = O.sample(logits, 0.5, context=ctx, **{k: v for k, v in okw.items() if k not in ("top_p", "min_p")})[1]
            c = np.cumsum(np.sort(base[op > 0])[::-1].astype(np.float64))
            assert abs(c[-1] - kw.get("top_p", 1.0)) < 2e-4 or abs(c[-2] - kw.get("top_p", 1.0)) < 2e-4
            continue
        assert np.abs(p - op).max() <= 2e-4 * max(op.max(), 1e-30), (u, np.abs(p - op).max())
        cdf = np.cumsum(op.astype(np.float64))
        if np.min(np.abs(cdf - u)) > 2e-4:
            assert tok == otok, (u, tok, otok)


def test_stream_read_runs_and_checks_its_size(gpu):
    """smx_stream_read (the bench's streaming-read ceiling) reads device memory without writing
    it, and refuses sizes that are not a positive multiple of 16 bytes."""
    import torch

    from smallmind_amd._lib import SmxError, call
    buf = torch.arange(1 << 18, dtype=torch.int32, device="cuda")
    before = buf.clone()
    s = torch.cuda.current_stream().cuda_stream
    for n in (16, 4096, buf.numel() * 4):
        call("smx_stream_read", buf.data_ptr(), n, s)
    torch.cuda.synchronize()
    assert torch.equal(buf, before)
    for n in (0, 24, 4095):
        with pytest.raises(SmxError):
            call("smx_stream_read", buf.data_ptr(), n, s)
