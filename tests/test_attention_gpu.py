"""GPU parity of paged split-KV decode attention against the oracle.

Bar (stated by the path's contract): fp16 outputs within max-abs 2e-3 and
rel 1e-2 of torch's CPU eager SDPA in fp32 over the gathered pages.  The
check is |gpu - ref| <= ATOL + RTOL * |ref| elementwise.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from tests.conftest import SEED

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL = 1e-2


def assert_close(got: torch.Tensor, ref: torch.Tensor):
    got = got.float().cpu()
    ref = ref.float().cpu()
    assert got.shape == ref.shape
    err = (got - ref).abs()
    bound = ATOL + RTOL * ref.abs()
    bad = err > bound
    assert not torch.isnan(got).any(), "NaN in output"
    assert not torch.isnan(ref).any(), "NaN in the reference"
    assert not bad.any(), f"{int(bad.sum())} elements out of tolerance; max abs err {err.max():.3e}"


def make_case(cuda, B, Hq, Hkv, D, ctx_lens, seed, extra_pages=3):
    """Random paged cache (device layout, filled directly on the GPU), a
    seeded random permutation of the page pool as block table, and q."""
    import torch_spyre_amd as tsa

    n_pages = [max(1, (c + 63) // 64) for c in ctx_lens]
    W = max(n_pages)
    pool = sum(n_pages) + extra_pages
    g = torch.Generator(device="cpu").manual_seed(seed)
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    table = torch.full((B, W), -1, dtype=torch.int32)
    k = 0
    for b, n in enumerate(n_pages):
        table[b, :n] = perm[k:k + n]
        k += n
    gg = torch.Generator(device=cuda).manual_seed(seed)
    cache = tsa.PagedKVCache(pool, Hkv, D, device=cuda, zero=False)
    cache.k.normal_(generator=gg)
    cache.v.normal_(generator=gg)
    q = torch.randn((B, Hq, D), generator=gg, device=cuda, dtype=torch.float32).half()
    lens = torch.tensor(ctx_lens, dtype=torch.int32)
    return cache, table, lens, q


def oracle_rows(cache, table, lens, q, rows, scale):
    """Gathers only the pages the sampled rows use, converts them to logical
    pages with the oracle's D2H, and runs torch CPU SDPA in fp32."""
    table = table.cpu().numpy()
    used = sorted({int(p) for b in rows for p in table[b][: max(1, (int(lens[b]) + 63) // 64)]})
    remap = {p: i for i, p in enumerate(used)}
    idx = torch.tensor(used, dtype=torch.long, device=cache.k.device)
    kd = cache.k.index_select(0, idx).cpu().numpy()
    vd = cache.v.index_select(0, idx).cpu().numpy()
    k_log, v_log = OA.pages_to_logical(kd, vd, len(used), cache.Hkv, cache.D)
    sub = np.full_like(table, -1)
    for b in rows:
        n = max(1, (int(lens[b]) + 63) // 64)
        sub[b, :n] = [remap[int(p)] for p in table[b][:n]]
    return OA.paged_decode_reference(q.cpu().float(), k_log, v_log, sub, lens.numpy(), scale, rows=rows)


def oracle_lse64(cache, table, lens, q, rows, scale):
    """fp64 logsumexp of scale q.k over each sampled row's tokens ([len(rows), Hq])."""
    tab = table.cpu().numpy()
    out = []
    for b in rows:
        n = max(1, (int(lens[b]) + 63) // 64)
        idx = torch.tensor([int(p) for p in tab[b][:n]], dtype=torch.long, device=cache.k.device)
        kd = cache.k.index_select(0, idx).cpu().numpy()
        k_log, v_log = OA.pages_to_logical(kd, np.zeros_like(kd).reshape(-1), n, cache.Hkv, cache.D)
        kb, _ = OA.gather_sequence(k_log, v_log, np.arange(n), int(lens[b]))
        out.append(OA.decode_lse_fp64(q[b].cpu().numpy(), kb, scale=scale))
    return np.stack(out)


def mean_v64(cache, table, lens, Hq, rows):
    """fp64 mean of V over each row's tokens, per q head ([len(rows), Hq, D]):
    the attention output when every score is equal (q = 0)."""
    tab = table.cpu().numpy()
    out = []
    for b in rows:
        n = max(1, (int(lens[b]) + 63) // 64)
        idx = torch.tensor([int(p) for p in tab[b][:n]], dtype=torch.long, device=cache.v.device)
        vd = cache.v.index_select(0, idx)
        _, v_log = OA.pages_to_logical(torch.zeros_like(vd).cpu().numpy(), vd.cpu().numpy(), n, cache.Hkv, cache.D)
        _, vb = OA.gather_sequence(v_log, v_log, np.arange(n), int(lens[b]))
        m = vb.astype(np.float64).mean(axis=1)  # [Hkv, D]
        out.append(np.repeat(m, Hq // cache.Hkv, axis=0))
    return np.stack(out)


def assert_token_count_exact(out, lse, ref_mean, lens, rows):
    """q = 0: every score is 0, P = 1 exactly and the row sum is exactly the
    number of visible tokens, so LSE = ln(n) up to fp32 rounding of the log
    (bound 4e-6, below ln(n / (n - 1)) for every n <= 131073) and out =
    mean(V) up to its fp16 rounding (half an fp16 ulp + 1e-6; a lost or
    doubled token moves some element of the mean by |v_t - mean| / n, several
    fp16 ulps for the largest of the 128 * Hq features)."""
    for i, b in enumerate(rows):
        n = int(lens[b])
        err = np.abs(lse[b].cpu().numpy().astype(np.float64) - math.log(n)).max()
        assert err <= 4e-6 < math.log(n / (n - 1)), (b, n, err)
        got = out[b].float().cpu().numpy().astype(np.float64)
        ref = ref_mean[i]
        # the spacing above |ref| (at a power of two the wider of the two binades)
        tol = 0.5 * np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64) + 1e-6
        bad = np.abs(got - ref) > tol
        assert not bad.any(), (b, n, int(bad.sum()), float(np.abs(got - ref).max()))


def run(cache, table, lens, q, cuda, **kw):
    import torch_spyre_amd as tsa

    return tsa.paged_decode_attention(q, cache.k, cache.v, table.to(cuda), lens.to(cuda), **kw)


def test_config1_dense_mha_vs_cpu_sdpa(cuda):
    """B=1, 8 heads MHA, D=64, ctx 512, contiguous fp16 q/k/v ~ N(0,1), scale 1/8."""
    import torch_spyre_amd as tsa

    g = torch.Generator().manual_seed(SEED)
    q = torch.randn((1, 8, 1, 64), generator=g).half()
    k = torch.randn((1, 8, 512, 64), generator=g).half()
    v = torch.randn((1, 8, 512, 64), generator=g).half()
    out = tsa.sdpa_decode(q.to(cuda), k.to(cuda), v.to(cuda), scale=0.125)
    ref = OA.sdpa_cpu_fp32(q, k, v, scale=0.125)
    assert_close(out, ref)
    ref64 = torch.from_numpy(OA.sdpa_decomposition_fp64(q.numpy(), k.numpy(), v.numpy(), 0.125))
    assert_close(out, ref64)


def test_config1_token_count_exact(cuda):
    """Config 1 through the SDPA kernels with q = 0 (closed form): LSE =
    ln(512) and out = mean(V) over all 512 keys, for all 8 heads."""
    import torch_spyre_amd as tsa

    g = torch.Generator().manual_seed(SEED + 2)
    v = torch.randn((1, 8, 512, 64), generator=g).half()
    k = torch.randn((1, 8, 512, 64), generator=g).half()
    out, lse = tsa.scaled_dot_product_attention(torch.zeros((1, 8, 1, 64), dtype=torch.float16, device=cuda),
                                                k.to(cuda), v.to(cuda), scale=0.125, return_lse=True)
    assert np.abs(lse.cpu().numpy().astype(np.float64) - math.log(512)).max() <= 4e-6
    ref = v[0].double().mean(dim=1).numpy()  # [8, 64]
    got = out[0, :, 0].float().cpu().numpy().astype(np.float64)
    tol = 0.5 * np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64) + 1e-6
    assert (np.abs(got - ref) <= tol).all()


@pytest.mark.parametrize("S", [1, 65, 513])
@pytest.mark.parametrize("D", [64, 128])
def test_dense_to_pages_then_paged_decode(cuda, S, D):
    """Dense K/V moved into the page layouts by dense_to_pages (one relayout
    pass per tensor, tokens past S zero-filled), then the paged kernel."""
    import torch_spyre_amd as tsa

    g = torch.Generator().manual_seed(SEED + 7 * S + D)
    q = torch.randn((2, 8, 1, D), generator=g).half()
    k = torch.randn((2, 2, S, D), generator=g).half()
    v = torch.randn((2, 2, S, D), generator=g).half()
    cache, table = tsa.dense_to_pages(k.to(cuda), v.to(cuda))
    lens = torch.full((2,), S, dtype=torch.int32, device=cuda)
    out = tsa.paged_decode_attention(q[:, :, 0].contiguous().to(cuda), cache.k, cache.v, table, lens,
                                     max_context_len=S)
    assert_close(out.unsqueeze(2), OA.sdpa_cpu_fp32(q, k, v))


@pytest.mark.parametrize("S", [1, 63, 64, 65, 200, 513])
@pytest.mark.parametrize("D", [64, 128])
def test_dense_gqa_ragged_lengths(cuda, S, D):
    import torch_spyre_amd as tsa

    g = torch.Generator().manual_seed(SEED + S + D)
    q = torch.randn((2, 8, 1, D), generator=g).half()
    k = torch.randn((2, 2, S, D), generator=g).half()
    v = torch.randn((2, 2, S, D), generator=g).half()
    out = tsa.sdpa_decode(q.to(cuda), k.to(cuda), v.to(cuda), enable_gqa=True)
    assert_close(out, OA.sdpa_cpu_fp32(q, k, v))


def test_config3_llama3_8b_full(cuda):
    """Batch 32, 32 q / 8 KV heads, D 128, ctx 4096, 64-token pages in a
    permuted pool -- every row checked against the oracle."""
    B, Hq, Hkv, D, ctx = 32, 32, 8, 128, 4096
    cache, table, lens, q = make_case(cuda, B, Hq, Hkv, D, [ctx] * B, SEED)
    out, lse = run(cache, table, lens, q, cuda, max_context_len=ctx, return_lse=True)
    ref = oracle_rows(cache, table, lens, q, list(range(B)), 1 / math.sqrt(D))
    assert_close(out, ref)
    # fp64 LSE of every row, bound 1e-4: below ln(4096 / 4095) = 2.4e-4, the
    # shift one lost or doubled token of equal score would cause
    lse64 = oracle_lse64(cache, table, lens, q, list(range(B)), 1 / math.sqrt(D))
    assert np.abs(lse.cpu().numpy() - lse64).max() <= 1e-4 < math.log(4096 / 4095)


def test_config3_token_count_exact(cuda):
    """The Llama-3-8B shape with q = 0 (closed form): LSE = ln(4096) and
    out = mean(V) for all 32 sequences."""
    B, Hq, Hkv, D, ctx = 32, 32, 8, 128, 4096
    cache, table, lens, q = make_case(cuda, B, Hq, Hkv, D, [ctx] * B, SEED + 1)
    out, lse = run(cache, table, lens, torch.zeros_like(q), cuda, max_context_len=ctx, return_lse=True)
    rows = list(range(B))
    assert_token_count_exact(out, lse, mean_v64(cache, table, lens, Hq, rows), lens, rows)


@pytest.mark.parametrize("split", [256, 64])
@pytest.mark.parametrize("g", [1, 2, 4, 8, 16])
def test_gqa_groups(cuda, g, split):
    """Every group size up to the MFMA's 16 columns.  Split 256: each
    sequence is one chunk, finished by its workgroup (whose threads fold
    g x D output elements, several each when g > 4); split 64: chunks of 512
    tokens, so 700 and 1500 go through the chunk partials and the merge."""
    Hkv, D = 2, 128
    lens = [1, 64, 100, 700, 1500]
    cache, table, lens_t, q = make_case(cuda, len(lens), g * Hkv, Hkv, D, lens, SEED + g)
    out = run(cache, table, lens_t, q, cuda, split_tokens=split)
    ref = oracle_rows(cache, table, lens_t, q, list(range(len(lens))), 1 / math.sqrt(D))
    assert_close(out, ref)


@pytest.mark.parametrize("split", [512, 64])
def test_ragged_edges_and_empty(cuda, split):
    """Contexts at page, split and chunk boundaries, and an empty context
    (zeros, as torch's CPU SDPA returns).  Split 512: every sequence fits one
    chunk (one kernel); split 64: chunks of 512 tokens, merge pass for the
    longer sequences only."""
    lens = [0, 1, 63, 64, 65, 511, 512, 513, 1023, 1024, 1025, 4000]
    cache, table, lens_t, q = make_case(cuda, len(lens), 32, 8, 128, lens, SEED + 99)
    out, lse = run(cache, table, lens_t, q, cuda, return_lse=True, split_tokens=split)
    rows = [b for b, c in enumerate(lens) if c > 0]
    ref = oracle_rows(cache, table, lens_t, q, rows, 1 / math.sqrt(128))
    assert_close(out[rows], ref)
    assert torch.count_nonzero(out[0]) == 0
    assert torch.isinf(lse[0]).all()


def test_lse_matches_oracle(cuda):
    lens = [70, 900]
    cache, table, lens_t, q = make_case(cuda, 2, 8, 2, 64, lens, SEED + 5)
    scale = 0.3
    out, lse = run(cache, table, lens_t, q, cuda, scale=scale, return_lse=True)
    tab = table.numpy()
    k_log, v_log = OA.pages_to_logical(cache.k.cpu().numpy(), cache.v.cpu().numpy(), cache.num_pages, 2, 64)
    for b, c in enumerate(lens):
        kb, _ = OA.gather_sequence(k_log, v_log, tab[b], c)
        qb = q[b].cpu().double().numpy()  # [Hq, D]
        kk = np.repeat(kb.astype(np.float64), 4, axis=0)  # [Hq, c, D]
        s = scale * np.einsum("hd,htd->ht", qb, kk)
        want = np.log(np.exp(s - s.max(1, keepdims=True)).sum(1)) + s.max(1)
        assert np.allclose(lse[b].cpu().numpy(), want, atol=1e-3, rtol=1e-4)


def test_split_invariance(cuda):
    """Different split sizes (1 page .. whole context) agree within tolerance."""
    lens = [3000, 2049, 77]
    cache, table, lens_t, q = make_case(cuda, 3, 16, 4, 128, lens, SEED + 8)
    base = run(cache, table, lens_t, q, cuda, split_tokens=4096)
    for split in (64, 128, 512, 1024):
        assert_close(run(cache, table, lens_t, q, cuda, split_tokens=split), base)


def test_page_permutation_invariance_bitexact(cuda):
    """Moving pages to other physical slots (and updating the table) gives
    bit-identical output: the arithmetic follows logical token order only."""
    lens = [1000, 333]
    cache, table, lens_t, q = make_case(cuda, 2, 32, 8, 128, lens, SEED + 13)
    out1 = run(cache, table, lens_t, q, cuda)
    perm = torch.randperm(cache.num_pages, generator=torch.Generator().manual_seed(3))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(cache.num_pages)
    cache.k.copy_(cache.k[perm.to(cuda)].clone())
    cache.v.copy_(cache.v[perm.to(cuda)].clone())
    table2 = torch.where(table >= 0, inv[table.clamp(min=0).long()].to(torch.int32), table)
    out2 = run(cache, table2, lens_t, q, cuda)
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))


def _config4_lens():
    g = torch.Generator().manual_seed(SEED)
    return torch.randint(128, 32769, (64,), generator=g).tolist()


def test_config4_ragged_full_shape_all_rows(cuda):
    """64 sequences, ctx ~ U[128, 32768] (seeded), 32/8 heads, D 128, split
    512 (sequences over 4096 tokens go through the chunk partials and the
    merge); every row against the oracle, LSE against fp64 (1e-4)."""
    lens = _config4_lens()
    cache, table, lens_t, q = make_case(cuda, 64, 32, 8, 128, lens, SEED + 4)
    out, lse = run(cache, table, lens_t, q, cuda, split_tokens=512, max_context_len=max(lens), return_lse=True)
    rows = list(range(64))
    for lo in range(0, 64, 16):
        assert_close(out[lo:lo + 16], oracle_rows(cache, table, lens_t, q, rows[lo:lo + 16], 1 / math.sqrt(128)))
    lse64 = oracle_lse64(cache, table, lens_t, q, rows, 1 / math.sqrt(128))
    assert np.abs(lse.cpu().numpy() - lse64).max() <= 1e-4


def test_config4_token_count_exact(cuda):
    """The ragged batch with q = 0 (closed form): for every one of the 64
    sequences LSE = ln(ctx) and out = mean(V)."""
    lens = _config4_lens()
    cache, table, lens_t, q = make_case(cuda, 64, 32, 8, 128, lens, SEED + 5)
    out, lse = run(cache, table, lens_t, torch.zeros_like(q), cuda, split_tokens=512, max_context_len=max(lens),
                   return_lse=True)
    rows = list(range(64))
    assert_token_count_exact(out, lse, mean_v64(cache, table, lens_t, 32, rows), lens_t, rows)


def test_bad_page_id_gives_nan_not_fault(cuda):
    lens = [200]
    cache, table, lens_t, q = make_case(cuda, 1, 4, 1, 64, lens, SEED + 21)
    table[0, 1] = cache.num_pages + 1000  # out of range
    out = run(cache, table, lens_t, q, cuda)
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()


def test_argument_errors(cuda):
    import torch_spyre_amd as tsa

    cache, table, lens_t, q = make_case(cuda, 1, 6, 4, 64, [100], SEED)
    with pytest.raises(ValueError):
        run(cache, table, lens_t, q, cuda)  # 6 % 4 != 0
    cache, table, lens_t, q = make_case(cuda, 1, 4, 1, 64, [100], SEED)
    with pytest.raises(ValueError):
        run(cache, table, lens_t, q, cuda, max_context_len=10_000)  # table too short
    with pytest.raises(ValueError):
        run(cache, table, lens_t, q, cuda, workspace=torch.empty(4, dtype=torch.uint8, device=cuda))
    with pytest.raises(tsa._lib.SpyreHipError):
        run(cache, table, lens_t, q, cuda, split_tokens=100)


def test_host_tensors_refused_before_any_launch(cuda):
    """A tensor a kernel would reach through its pointer must be on the
    call's GPU: host (CPU) tensors in those places raise before anything is
    launched, in every entry point (the C++ operators, the ctypes calls, the
    prepared call and the two passes)."""
    import torch_spyre_amd as tsa

    cache, table, lens_t, q = make_case(cuda, 2, 8, 2, 64, [100, 300], SEED + 30)
    table, lens_t = table.to(cuda), lens_t.to(cuda)
    ws_dev = torch.empty(tsa.workspace_bytes(2, 8, 2, 64, 300), dtype=torch.uint8, device=cuda)
    ws_cpu = torch.empty(ws_dev.numel(), dtype=torch.uint8)
    with pytest.raises(ValueError, match="context_lens"):
        tsa.paged_decode_attention(q, cache.k, cache.v, table, lens_t.cpu(), max_context_len=300)
    with pytest.raises(ValueError, match="block_table"):
        tsa.paged_decode_attention(q, cache.k, cache.v, table.cpu(), lens_t, max_context_len=300)
    with pytest.raises(ValueError, match="workspace"):
        tsa.paged_decode_attention(q, cache.k, cache.v, table, lens_t, max_context_len=300, workspace=ws_cpu)
    with pytest.raises(ValueError, match="context_lens"):
        tsa.paged_decode_attention(q, cache.k, cache.v, table, lens_t.cpu(), max_context_len=300, workspace=ws_dev)
    with pytest.raises(ValueError, match="out"):
        tsa.paged_decode_attention(q, cache.k, cache.v, table, lens_t, max_context_len=300,
                                   out=torch.empty(q.shape, dtype=q.dtype))
    with pytest.raises(ValueError, match="out"):
        tsa.PagedDecode(q, cache.k, cache.v, table, lens_t, max_context_len=300, out=torch.empty(q.shape, dtype=q.dtype))
    with pytest.raises(ValueError, match="workspace"):
        tsa.paged_decode_merge(lens_t, ws_cpu, torch.empty_like(q), 2, 300)
    with pytest.raises(ValueError, match="positions"):
        tsa.kv_append(q[:, :2].contiguous(), q[:, :2].contiguous(), cache.k, cache.v, table,
                      torch.zeros(2, dtype=torch.int32))
    with pytest.raises(ValueError, match="block_table"):
        tsa.kv_append(q[:, :2].contiguous(), q[:, :2].contiguous(), cache.k, cache.v, table.cpu(),
                      torch.zeros(2, dtype=torch.int32, device=cuda))
    qs = torch.zeros((1, 2, 8, 64), dtype=torch.float16, device=cuda)
    with pytest.raises(ValueError, match="workspace"):
        tsa.scaled_dot_product_attention(qs, qs, qs, workspace=torch.empty(1 << 20, dtype=torch.uint8))
    torch.cuda.synchronize()


@pytest.mark.parametrize("lens", [[700, 64, 1999], [700, 64, 1999, 5000, 0, 2048, 2049]])
def test_two_pass_api_equals_single_call_bitexact(cuda, lens):
    """paged_decode_split + paged_decode_merge == paged_decode_attention,
    both when the single call is one kernel (every context fits one chunk of
    8 x 256 tokens) and when it merges the longer sequences only."""
    import torch_spyre_amd as tsa

    B = len(lens)
    cache, table, lens_t, q = make_case(cuda, B, 32, 8, 128, lens, SEED + 41)
    t, l = table.to(cuda), lens_t.to(cuda)
    ws = torch.empty(tsa.workspace_bytes(B, 32, 8, 128, max(lens), 256), dtype=torch.uint8, device=cuda)
    one, lse1 = tsa.paged_decode_attention(q, cache.k, cache.v, t, l, split_tokens=256,
                                           max_context_len=max(lens), return_lse=True)
    tsa.paged_decode_split(q, cache.k, cache.v, t, l, ws, split_tokens=256, max_context_len=max(lens))
    two = torch.empty_like(q)
    lse2 = torch.empty((B, 32), dtype=torch.float32, device=cuda)
    tsa.paged_decode_merge(l, ws, two, 8, max(lens), split_tokens=256, lse=lse2)
    assert torch.equal(one.view(torch.int16), two.view(torch.int16))
    assert torch.equal(lse1, lse2)


@pytest.mark.parametrize("B,kernels,D", [(7, 1, 128), (40, 2, 128), (7, 1, 64), (40, 2, 64)], ids=str)
def test_chunks_merge_in_kernel_or_pass(cuda, B, kernels, D):
    """Contexts of up to three 2048-token chunks (split 256).  7 sequences x
    8 KV heads x 3 chunks fit one round of a 256-CU device's workgroups, so
    the chunks merge inside the split kernel (one kernel); 40 sequences take
    four rounds and the merge pass.  Both bit-equal to the two-pass API
    (split, then the merge pass), every row against the oracle; D 128 and 64."""
    import torch_spyre_amd as tsa
    from torch_spyre_amd import _lib

    if torch.cuda.get_device_properties(cuda).multi_processor_count != 256:
        pytest.skip("the kernel counts assume a 256-CU device")
    lens = ([5000, 700, 64, 4097, 2049, 1, 6000] * 6)[:B]
    assert _lib.lib().spyre_paged_decode_attn_kernels(B, 32, 8, D, max(lens), 256) == kernels
    cache, table, lens_t, q = make_case(cuda, B, 32, 8, D, lens, SEED + 43 + B + D)
    t, l = table.to(cuda), lens_t.to(cuda)
    call = tsa.PagedDecode(q, cache.k, cache.v, t, l, split_tokens=256, max_context_len=max(lens),
                           lse=torch.empty((B, 32), dtype=torch.float32, device=cuda))
    assert call.passes == kernels
    one = call().clone()
    lse1 = call.lse.clone()
    call.split()
    two = call.merge()
    assert torch.equal(one.view(torch.int16), two.view(torch.int16))
    assert torch.equal(lse1, call.lse)
    rows = list(range(B))
    assert_close(one, oracle_rows(cache, table, lens_t, q, rows, 1 / math.sqrt(D)))


def test_workspace_alignment_paths_agree(cuda):
    """A 16-byte aligned workspace (two-chunk contexts merged inside the
    split kernel) and one 4 bytes off it (the merge pass with scalar loads)
    give the same bits, output and LSE; both against the oracle."""
    import torch_spyre_amd as tsa

    lens = [5000, 700, 64, 4097]
    B = len(lens)
    cache, table, lens_t, q = make_case(cuda, B, 32, 8, 128, lens, SEED + 49)
    t, l = table.to(cuda), lens_t.to(cuda)
    need = tsa.workspace_bytes(B, 32, 8, 128, max(lens), 256)
    buf = torch.empty(need + 64, dtype=torch.uint8, device=cuda)
    res = []
    for off in (0, 4):
        ws = buf[off:off + need]
        assert ws.data_ptr() % 16 == off
        res.append(tsa.paged_decode_attention(q, cache.k, cache.v, t, l, split_tokens=256, max_context_len=max(lens),
                                              workspace=ws, return_lse=True))
    assert torch.equal(res[0][0].view(torch.int16), res[1][0].view(torch.int16))
    assert torch.equal(res[0][1], res[1][1])
    assert_close(res[0][0], oracle_rows(cache, table, lens_t, q, list(range(B)), 1 / math.sqrt(128)))


@pytest.mark.parametrize("split", [512, 256])
def test_context_past_max_gives_nan_rows(cuda, split):
    """A context longer than max_context_len breaks the call's contract: the
    kernel reads only max_context_len tokens of it and its rows come out NaN,
    the others exact.  Split 512: every context one chunk (one kernel);
    split 256: two chunks merged inside the kernel; and the two-pass API."""
    import torch_spyre_amd as tsa

    lens = [5000, 700, 3000, 64]
    cache, table, lens_t, q = make_case(cuda, 4, 32, 8, 128, lens, SEED + 47)
    t, l = table.to(cuda), lens_t.to(cuda)
    out = tsa.paged_decode_attention(q, cache.k, cache.v, t, l, split_tokens=split, max_context_len=4000)
    ws = torch.empty(tsa.workspace_bytes(4, 32, 8, 128, 4000, split), dtype=torch.uint8, device=cuda)
    tsa.paged_decode_split(q, cache.k, cache.v, t, l, ws, split_tokens=split, max_context_len=4000)
    two = tsa.paged_decode_merge(l, ws, torch.empty_like(q), 8, 4000, split_tokens=split)
    for o in (out, two):
        assert torch.isnan(o[0].float()).all()
        assert_close(o[1:], oracle_rows(cache, table, lens_t, q, [1, 2, 3], 1 / math.sqrt(128)))


def test_prepared_call_matches(cuda):
    """PagedDecode (validated once, launched repeatedly) == paged_decode_attention."""
    import torch_spyre_amd as tsa

    lens = [300, 1200]
    cache, table, lens_t, q = make_case(cuda, 2, 16, 4, 128, lens, SEED + 51)
    t, l = table.to(cuda), lens_t.to(cuda)
    want = tsa.paged_decode_attention(q, cache.k, cache.v, t, l, max_context_len=max(lens))
    call = tsa.PagedDecode(q, cache.k, cache.v, t, l, max_context_len=max(lens))
    for _ in range(3):
        got = call()
    assert torch.equal(want.view(torch.int16), got.view(torch.int16))


def test_large_batch_grid_mode(cuda):
    """Batches over 1024 sequences take the grid-mode split kernel; sampled
    rows (including empty and one-token contexts, and contexts of up to three
    512-token chunks) against the oracle."""
    g = torch.Generator().manual_seed(SEED + 61)
    B = 1100
    lens = torch.randint(0, 1200, (B,), generator=g).tolist()
    lens[0], lens[1], lens[2] = 0, 1, 1199
    cache, table, lens_t, q = make_case(cuda, B, 8, 2, 64, lens, SEED + 62)
    out = run(cache, table, lens_t, q, cuda, split_tokens=64)
    rows = [1, 2, 5, 500, 777, B - 1]
    rows = [r for r in rows if lens[r] > 0]
    assert_close(out[rows], oracle_rows(cache, table, lens_t, q, rows, 1 / math.sqrt(64)))
    assert torch.count_nonzero(out[0]) == 0


def test_workspace_reuse_across_shapes(cuda):
    """One workspace reused by calls of different shapes (partials left over
    from earlier calls) gives the same bits as a fresh workspace each time."""
    import torch_spyre_amd as tsa

    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=cuda)
    shapes = [(3, 32, 8, 128, [1000, 70, 2200]), (5, 8, 2, 64, [64, 65, 1, 3000, 512]),
              (3, 32, 8, 128, [1000, 70, 2200]), (2, 16, 16, 128, [4000, 10])]
    for i, (B, Hq, Hkv, D, lens) in enumerate(shapes):
        cache, table, lens_t, q = make_case(cuda, B, Hq, Hkv, D, lens, SEED + 70 + i)
        t, l = table.to(cuda), lens_t.to(cuda)
        reused = tsa.paged_decode_attention(q, cache.k, cache.v, t, l, split_tokens=128,
                                            max_context_len=max(lens), workspace=ws)
        fresh = tsa.paged_decode_attention(q, cache.k, cache.v, t, l, split_tokens=128,
                                           max_context_len=max(lens))
        assert torch.equal(reused.view(torch.int16), fresh.view(torch.int16)), i


def test_balanced_chunks_fill_rounds(cuda):
    """32 sequences x 8 KV heads of 9 pages at split 64 (8-page chunks): two
    chunks per (sequence, KV head) would make 512 split workgroups, two rounds
    on a 256-slot device (256 CUs, one 8-wavefront workgroup each), so the
    planner grows the chunk to 9 pages and every pair is one chunk.  All rows
    against the oracle; the two-pass API (whose merge then finds only single
    chunks) gives the same bits; and on a 256-CU device the result equals
    split 512 bit for bit (both cut each context into one chunk the same way)."""
    import torch_spyre_amd as tsa

    B, Hq, Hkv, D = 32, 32, 8, 128
    lens = [576] * B
    lens[3], lens[17], lens[31] = 513, 100, 0
    cache, table, lens_t, q = make_case(cuda, B, Hq, Hkv, D, lens, SEED + 81)
    t, l = table.to(cuda), lens_t.to(cuda)
    out, lse = tsa.paged_decode_attention(q, cache.k, cache.v, t, l, split_tokens=64, max_context_len=576,
                                          return_lse=True)
    rows = [b for b in range(B) if lens[b] > 0]
    assert_close(out[rows], oracle_rows(cache, table, lens_t, q, rows, 1 / math.sqrt(D)))
    assert torch.count_nonzero(out[31]) == 0
    ws = torch.empty(tsa.workspace_bytes(B, Hq, Hkv, D, 576, 64), dtype=torch.uint8, device=cuda)
    tsa.paged_decode_split(q, cache.k, cache.v, t, l, ws, split_tokens=64, max_context_len=576)
    two = torch.empty_like(q)
    lse2 = torch.empty((B, Hq), dtype=torch.float32, device=cuda)
    tsa.paged_decode_merge(l, ws, two, Hkv, 576, split_tokens=64, lse=lse2)
    assert torch.equal(out.view(torch.int16), two.view(torch.int16))
    assert torch.equal(lse, lse2)
    if torch.cuda.get_device_properties(cuda).multi_processor_count == 256:
        wide = tsa.paged_decode_attention(q, cache.k, cache.v, t, l, split_tokens=512, max_context_len=576)
        assert torch.equal(out.view(torch.int16), wide.view(torch.int16))
