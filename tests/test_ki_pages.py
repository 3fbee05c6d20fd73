"""The KI page image (pd_vllm/profiles/mla_nsa.py:17-41,211-228) built on the host, and
the paged entry points' argument checks.  CPU only."""
import torch

from tilert_amd import sparse_index as si


def test_page_constants_match_the_reference_format():
    # PAGE_SIZE = 64; KI_PAGE_BYTES = 64*128 + 64*128//128*4 = 8448 (mla_nsa.py:22-41)
    assert si.KI_PAGE_KEYS == 64 and si.KI_PAGE_BYTES == 8448


def test_ki_pages_from_flat_layout():
    L = 130
    g = torch.Generator().manual_seed(0)
    raw = torch.randint(0, 256, (L, 128), generator=g, dtype=torch.uint8)
    raw[raw == 0x7f] = 0  # keep clear of NaN codes so the fp8 view compares cleanly
    raw[raw == 0xff] = 0
    kv = raw.view(torch.float8_e4m3fn)
    ks = torch.rand(L, generator=g) + 0.1
    pages = si.ki_pages_from_flat(kv, ks)
    assert pages.shape == (3, 8448) and pages.dtype == torch.uint8
    for key in (0, 63, 64, 100, 129):
        p, r = divmod(key, 64)
        assert torch.equal(pages[p, r * 128:(r + 1) * 128], raw[key])
        sc = pages[p, 8192 + 4 * r: 8192 + 4 * (r + 1)].view(torch.float32)[0]
        assert sc.item() == ks[key].item()
    # rows past L are zero: fp8 bytes and scales
    assert torch.all(pages[2, 2 * 128:8192] == 0)
    assert torch.all(pages[2, 8192 + 2 * 4:] == 0)


def test_paged_entry_points_check_arguments_without_a_gpu():
    from tilert_amd import _lib
    lib = _lib.load()
    # 65 keys do not fit one page
    assert lib.tl_indexer_fp8_scores_paged(None, None, 0, None, 1, None, None, 4, 64, 65, 65, 60, None) == 1
    assert b"pages" in lib.tl_last_error()
    assert lib.tl_indexer_fp8_scores_paged(None, None, 0, None, 2, None, None, 4, 64, 65, 65, 60, None) == 1
    assert b"null pointer" in lib.tl_last_error()
    assert lib.tl_ki_cache_write(None, 10, None, 1, 60, 2, None) == 1
    assert b"exceed" in lib.tl_last_error()
    assert lib.tl_ki_cache_write(None, 10, None, 1, 0, 5, None) == 1
    assert b"scale_mode" in lib.tl_last_error()
