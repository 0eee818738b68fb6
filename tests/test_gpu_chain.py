"""GPU checks of the chained expert GEMMs (camhipMoeExperts): GMM1 + SwiGLU and GMM2 in one launch, each
GMM2 tile waiting for the GMM1 tiles of its rows through per-M-tile readiness counters.

The chained launch must be bit-identical to the two grouped-matmul calls it replaces (h, its fp8 scales and
the bf16 output), on repeated calls and on HIP-graph replays, and its bounded wait must give up cleanly when
the host makes every target unreachable (camhipDebugSetSyncWait): the launch ends normally and the device's
sync status reports it.  The two-call path itself is checked against the oracle in test_gpu_gmm.py."""
import pytest
import torch

pytestmark = pytest.mark.gpu

QUANT_NONE, QUANT_FP8 = 0, 3
DT_BF16, DT_FP8 = 0, 3


@pytest.fixture(scope="module")
def lib():
    import umdk_amd  # noqa: F401
    from umdk_amd import _lib
    return _lib


def fp8_quant_rows_kmajor(x):
    """1x128 fp8 quantisation of [m, k] rows; scales returned k-major as a [k/128, m] tensor."""
    m, k = x.shape
    xv = x.float().view(m, k // 128, 128)
    amax = xv.abs().amax(2).clamp(min=1e-4)
    q = (xv * torch.div(torch.full_like(amax, 448.0), amax).unsqueeze(2)).to(torch.float8_e4m3fn)
    return q.view(m, k), torch.div(amax, torch.full_like(amax, 448.0)).t().contiguous()


def fp8_quant_weight(w):
    L, n, k = w.shape
    wv = w.float().view(L, n // 128, 128, k // 128, 128)
    amax = wv.abs().amax(dim=(2, 4)).clamp(min=1e-6)
    q = (wv / (amax / 448.0)[:, :, None, :, None]).to(torch.float8_e4m3fn)
    return q.view(L, n, k), (amax / 448.0).contiguous()


class Case:
    """Inputs of one expert layer's GEMMs on the GPU, and output buffers for both paths."""

    def __init__(self, counts, H, I, dt, seed):
        g = torch.Generator(device="cuda").manual_seed(seed)
        self.L, self.M, self.H, self.I, self.dt = len(counts), sum(counts), H, I, dt
        self.cap = self.M + 5  # rows past the groups: never read as a group row, never written
        dev = "cuda"
        self.gl = torch.tensor(counts, dtype=torch.int64, device=dev)
        x = torch.randn(self.cap, H, device=dev, generator=g)
        w1 = torch.randn(self.L, 2 * I, H, device=dev, generator=g) * 0.03
        w2 = torch.randn(self.L, H, I, device=dev, generator=g) * 0.03
        if dt == DT_FP8:
            self.x, self.xs = fp8_quant_rows_kmajor(x)
            self.w1, self.w1s = fp8_quant_weight(w1)
            self.w2, self.w2s = fp8_quant_weight(w2)
        else:
            self.x, self.xs = x.bfloat16(), None
            self.w1, self.w1s, self.w2, self.w2s = w1.bfloat16(), None, w2.bfloat16(), None
        self.new_outputs()

    def new_outputs(self):
        hdt = torch.float8_e4m3fn if self.dt == DT_FP8 else torch.bfloat16
        out = {}
        for tag in ("pair", "chain"):
            h = torch.full((self.cap, self.I), 7, dtype=torch.uint8 if self.dt == DT_FP8 else torch.int16,
                           device="cuda").view(hdt)
            hs = torch.full((self.I // 128, self.cap), -1.0, device="cuda") if self.dt == DT_FP8 else None
            y = torch.full((self.cap, self.H), 3, dtype=torch.int16, device="cuda").view(torch.bfloat16)
            out[tag] = (h, hs, y)
        self.out = out

    @staticmethod
    def p(t):
        return None if t is None else t.data_ptr()

    def run_pair(self, lib):
        h, hs, y = self.out["pair"]
        p = self.p
        lib.call("camhipGroupedMatmulSwiglu", p(self.x), p(self.xs), p(self.gl), self.L, self.cap, self.H,
                 2 * self.I, p(self.w1), p(self.w1s), self.dt, 1, QUANT_FP8 if self.dt == DT_FP8 else QUANT_NONE,
                 p(h), p(hs), device="cuda")
        lib.call("camhipGroupedMatmul", p(h), p(hs), p(self.gl), self.L, self.cap, self.I, self.H, p(self.w2),
                 p(self.w2s), self.dt, 1, p(y), device="cuda")

    def chain_args(self):
        h, hs, y = self.out["chain"]
        p = self.p
        return (p(self.x), p(self.xs), p(self.gl), self.L, self.cap, self.H, 2 * self.I, p(self.w1), p(self.w1s),
                p(self.w2), p(self.w2s), self.dt, 1, p(h), p(hs), p(y))

    def run_chain(self, lib, workspace=None):
        if workspace is None:
            lib.call("camhipMoeExperts", *self.chain_args(), device="cuda")
        else:
            lib.launch("camhipMoeExperts", *self.chain_args(), workspace=workspace, device="cuda")

    def assert_same(self):
        torch.cuda.synchronize()
        M = self.M
        (h0, hs0, y0), (h1, hs1, y1) = self.out["pair"], self.out["chain"]
        u = lambda t: t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t.view(torch.int16)
        assert torch.equal(u(h0)[:M], u(h1)[:M]), "h differs between the chained and the two-call path"
        if hs0 is not None:
            assert torch.equal(hs0[:, :M], hs1[:, :M]), "h scales differ"
        assert torch.equal(y0.view(torch.int16)[:M], y1.view(torch.int16)[:M]), "GMM2 output differs"


def decode_counts(L=32, T=128, K=8, E=256, seed=0):
    """Rows per local expert of a decode step: routing of T tokens over E experts (top-K of N(0,1) logits),
    the ids below L kept (a rank's share of the experts)."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.randn(T, E, generator=g).topk(K, dim=1).indices
    return torch.bincount(ids[ids < L], minlength=L).tolist()


CASES = [
    # config 5's GEMM shapes: 32 local experts of DeepSeek-V3, decode rows
    (decode_counts(), 7168, 2048, DT_FP8),
    # ragged small groups, an empty one, rows past the groups
    ([3, 40, 0, 7], 1024, 256, DT_FP8),
    ([3, 40, 0, 7], 1024, 256, DT_BF16),
    # 512 groups, mostly empty (the readiness counters of the last experts)
    ([0] * 5 + [9] + [0] * 250 + [48, 1] + [0] * 253 + [2], 512, 128, DT_FP8),
    # every group at the 48-row average limit of the chained kernel, several tiles per group
    ([48] * 16, 2048, 1024, DT_FP8),
    ([45, 0, 48, 31, 47, 12, 48, 48], 2048, 1024, DT_BF16),
    # prefill-sized groups (the 8-wave chained kernel): config 4's skew -- four heavy experts on 256-row tiles,
    # light ones on 32-row tiles run by four of the eight waves
    ([1226, 725, 643, 482] + [62, 46, 30, 21, 17, 9, 7, 5, 4, 3, 2, 2, 1, 1, 1, 1] + [0] * 12, 7168, 2048, DT_FP8),
    # all three classes (256-, 128- and 32-row tiles) in both GEMMs
    ([400, 100, 30, 0, 1000, 64, 63, 5], 2048, 2048, DT_FP8),
    ([400, 100, 30, 0, 900, 64, 63, 5], 1024, 1024, DT_BF16),
    # short reductions: the 128-row class only
    ([100, 300, 5, 0, 700, 64, 63], 1024, 512, DT_FP8),
    # GEMMs that would split the experts differently (GMM1 256-row tiles, GMM2 128-row): the two calls
    ([400, 100, 30, 0, 1000, 64, 63, 5], 2048, 1024, DT_FP8),
]


@pytest.mark.parametrize("counts,H,I,dt", CASES)
def test_chain_matches_two_calls(lib, counts, H, I, dt):
    print(f"chain vs pair: L={len(counts)} M={sum(counts)} H={H} I={I} dt={dt}", flush=True)
    c = Case(counts, H, I, dt, seed=len(counts) + H + I)
    c.run_pair(lib)
    for rep in range(3):  # consecutive calls, each clearing its own counters
        c.run_chain(lib)
        c.assert_same()
        c.out["chain"][2].fill_(0.5)
    assert lib.sync_status() == 0


@pytest.mark.parametrize("counts", [decode_counts(seed=3), [1100, 700, 500, 3, 40, 0, 17, 9]])
def test_chain_graph_replays(lib, counts):
    """The chained call captured in a HIP graph: every replay, with eager work and a reset of the outputs
    between replays, equals the two-call path."""
    print(f"chain graph replays: fp8 H=7168 I=2048 M={sum(counts)}", flush=True)
    c = Case(counts, 7168, 2048, DT_FP8, seed=11)
    c.run_pair(lib)
    ws = torch.empty(lib.workspace_size("camhipMoeExperts", *c.chain_args()), dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        c.run_chain(lib, ws)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        c.run_chain(lib, ws)
    for rep in range(4):
        h, hs, y = c.out["chain"]
        h.view(torch.uint8).fill_(0x55)
        hs.fill_(-2.0)
        y.fill_(1.25)
        c.run_pair(lib)  # eager work between replays
        graph.replay()
        c.assert_same()
    del graph
    assert lib.sync_status() == 0


@pytest.mark.parametrize("counts,H,I", [([3, 40, 0, 7, 25], 1024, 256), ([400, 100, 30, 0, 1000, 64, 63, 5], 2048, 2048)])
def test_chain_wait_gives_up_when_unreachable(lib, counts, H, I):
    """Host-forced give-up: with every readiness target unreachable and a 20 us bound, each wait gives up,
    the launch ends normally and the sync status is set; a normal call afterwards is exact again."""
    print(f"chain forced give-up: fp8 M={sum(counts)} H={H} I={I}", flush=True)
    c = Case(counts, H, I, DT_FP8, seed=5)
    c.run_pair(lib)
    torch.cuda.synchronize()
    lib.sync_status(clear=True)
    L = lib.lib()
    L.camhipDebugSetSyncWait(2000, 1)  # 2000 ticks of the 100 MHz clock
    try:
        c.run_chain(lib)
        torch.cuda.synchronize()
    finally:
        L.camhipDebugSetSyncWait(0, 0)
    assert lib.sync_status(clear=True) != 0, "an unreachable wait did not report"
    assert lib.sync_status() == 0, "the status was not cleared"
    c.run_chain(lib)
    c.assert_same()
    assert lib.sync_status() == 0
