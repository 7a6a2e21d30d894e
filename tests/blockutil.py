"""Helpers shared by the GPU block tests: random block weights drawn on the
GPU, array comparison metrics, and the kernel-choice rules of the library's
linear dispatcher that a test composition has to mirror."""
import numpy as np
import torch

DEV = "cuda:0"
LINEAR_SHAPES = {"img_mod": (18432, 3072), "txt_mod": (18432, 3072)}
for _n in ("to_q", "to_k", "to_v", "add_q_proj", "add_k_proj", "add_v_proj", "to_out", "to_add_out"):
    LINEAR_SHAPES[_n] = (3072, 3072)
for _s in ("img", "txt"):
    LINEAR_SHAPES[f"{_s}_mlp_fc1"] = (12288, 3072)
    LINEAR_SHAPES[f"{_s}_mlp_fc2"] = (3072, 12288)
NORMS = ("norm_q", "norm_k", "norm_added_q", "norm_added_k")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def bf16_dev(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(DEV).view(torch.bfloat16)


def metrics(a, b):
    """(max|a-b| / max|b|, cosine similarity) in float64."""
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    rel = np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30)
    cos = float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))
    return rel, cos


def gpu_block(qimg, seed, mode=0):
    """Random N(0,0.02) block weights (bf16, quantized by the library) and
    N(0,0.01) biases drawn on the GPU; RMSNorm weights 1 + N(0,0.1)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    W = {n: qimg.quantize_weight_tensor((torch.randn(N, K, generator=g, device=DEV) * 0.02).to(torch.bfloat16),
                                        mode=mode) for n, (N, K) in LINEAR_SHAPES.items()}
    B = {n: (torch.randn(N, generator=g, device=DEV) * 0.01).to(torch.bfloat16)
         for n, (N, K) in LINEAR_SHAPES.items()}
    nr = {n: (1 + 0.1 * torch.randn(128, generator=g, device=DEV)).to(torch.bfloat16) for n in NORMS}
    return W, B, nr


def oracle_entries(W, B):
    """The oracle's (w_q, w_scales, hbs, bias_bits, mode) for each linear."""
    h = lambda t: t.cpu().numpy()
    return {n: (h(w.data).view(np.uint8) if w.mode == 1 else h(w.data), h(w.scales), w.had_block_size,
                h(B[n].view(torch.int16)).view(np.uint16), w.mode) for n, w in W.items()}


def large_tiles(M, N):
    return ((M + 255) // 256) * ((N + 255) // 256)


def cu_count():
    return torch.cuda.get_device_properties(0).multi_processor_count


# the dispatcher's small-M threshold (kSmallMTileLimit): linears with fewer
# 256x256 tiles than this run on the 64x64 tiles
SMALL_M_TILE_LIMIT = 64


def pair_in_one_launch(Ma, Na, Mb, Nb, cus):
    """Whether the dispatcher runs two e4m3 linears (image and text stream)
    in one launch of the large-tile kernel: the first needs at least
    SMALL_M_TILE_LIMIT tiles (below that the small-tile kernel takes it), the
    second's tiles must fit the first's last round, and the first must not be
    a case for the tail-row split (a last round less than half full)."""
    if min(Ma, Na, Mb, Nb) <= 0 or Ma <= 32 or large_tiles(Ma, Na) < SMALL_M_TILE_LIMIT:
        return False
    ta, tb = large_tiles(Ma, Na), large_tiles(Mb, Nb)
    rounds = (ta + cus - 1) // cus
    tail = ta - (rounds - 1) * cus
    return ta + tb <= rounds * cus and not (rounds > 1 and 2 * tail < cus)
