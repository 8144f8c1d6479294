"""snl_pick_rows_noalloc (the greedy pick with its block partials in a static device array)
against snl_pick_rows, through the C ABI: two calls in a row, the second smaller, each bitwise
equal to the allocating entry point and to the first index of the row maximum."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_pick_rows_noalloc_matches_pick_rows():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import snl
    from snl.engine import SNL_EARG, SnlError, kernels

    snl.lib()
    r = np.random.default_rng(41)
    for V, rows in ((248320, 2), (4096, 1)):
        print(f"pick V={V} rows={rows}", flush=True)
        lg = r.standard_normal((rows, V)).astype(np.float32)
        lg[0, V // 3] = lg[0, V - 5] = 9.0  # tie: the first index wins
        dl = torch.from_numpy(lg).cuda()
        ref = torch.zeros((rows, 4), dtype=torch.int32, device="cuda")
        got = torch.full((rows, 4), -1, dtype=torch.int32, device="cuda")
        kernels.pick_rows(dl, V, rows, ref)
        kernels.pick_rows_noalloc(dl, V, rows, got)
        torch.cuda.synchronize()
        a, b = ref.cpu().numpy(), got.cpu().numpy()
        assert np.array_equal(a, b)
        tok = b[:, 0].view(np.uint32)
        top = b[:, 1:3].view(np.float32)
        assert tok[0] == V // 3 and top[0, 0] == 9.0 and top[0, 1] == 9.0
        for i in range(rows):
            assert tok[i] == int(np.argmax(lg[i]))
    # past the static array's 4096 block partials: refused before any launch
    big = torch.zeros((34, 248320), dtype=torch.float32, device="cuda")
    picks = torch.zeros((34, 4), dtype=torch.int32, device="cuda")
    with pytest.raises(SnlError) as ei:
        kernels.pick_rows_noalloc(big, 248320, 34, picks)
    assert ei.value.code == SNL_EARG
