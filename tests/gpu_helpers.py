"""Helpers shared by the GPU parity tests: move oracle cases to the device in
the reference's pool layout and compare with the stated tolerances."""
import torch

# Attention tolerance against an fp32 (or fp64) reference, bf16 outputs.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def assert_close_attn(out, ref, what=""):
    """max-abs < 2e-2 and mean-abs < 2e-3 against an fp32/fp64 reference;
    prints the achieved errors so the margin to the bar is in the log."""
    d = (out.double().cpu() - ref.double().cpu()).abs()
    assert torch.isfinite(out.float()).all(), f"{what}: non-finite output"
    mx, mn = d.max().item(), d.mean().item()
    print(f"[err] {what}: max-abs {mx:.3e} (bar {MAX_ABS:.0e}), mean-abs {mn:.3e} "
          f"(bar {MEAN_ABS:.0e})", flush=True)
    assert mx < MAX_ABS and mn < MEAN_ABS, f"{what}: max-abs {mx:.3e} mean-abs {mn:.3e}"
    return mx, mn


def decode_case_to_device(case, dev, num_layers=2, layer=1, extra_rows=0):
    """Places the case's single-layer pool at `layer` of a layer-interleaved
    (num_blocks, num_layers, Hkv, bs, D) pool, as KVCachePool stores it, and
    returns the per-layer views plus device tables.  With extra_rows the
    resident table has unused rows (-1) after the batch rows."""
    nb, hkv, bs, d = case.k_pool.shape
    kfull = torch.zeros(nb, num_layers, hkv, bs, d, dtype=torch.bfloat16, device=dev)
    vfull = torch.zeros_like(kfull)
    kfull[:, layer] = case.k_pool.to(dev)
    vfull[:, layer] = case.v_pool.to(dev)
    B, mp = case.block_table.shape
    bt = torch.full((B + extra_rows, mp), -1, dtype=torch.int32, device=dev)
    bt[:B] = case.block_table.to(dev)
    sl = torch.zeros(B + extra_rows, dtype=torch.int32, device=dev)
    sl[:B] = case.seq_lens.to(dev)
    return dict(q=case.q.to(dev), k=kfull[:, layer], v=vfull[:, layer], kfull=kfull,
                vfull=vfull, bt=bt, seq_lens=sl, row_ids=case.row_ids.to(dev))


def gpu_dense_decode_fp32(q, k_layer, v_layer, bt, seq_lens, row_ids, block_size, bias=1):
    """fp32 torch reference on the GPU (gather through the table, plain
    softmax) for workloads too large for the CPU oracle."""
    B, H, D = q.shape
    Hk = k_layer.shape[1]
    G = H // Hk
    out = torch.empty(B, H, D, dtype=torch.float32, device=q.device)
    rows = row_ids.tolist() if row_ids is not None else list(range(B))
    lens = (seq_lens.cpu().long() + bias).tolist()
    bt_cpu = bt.cpu()
    for b, row in enumerate(rows):
        L = lens[row]
        n = (L + block_size - 1) // block_size
        pages = bt_cpu[row, :n].long().to(q.device)
        kc = k_layer[pages].permute(1, 0, 2, 3).reshape(Hk, n * block_size, D)[:, :L].float()
        vc = v_layer[pages].permute(1, 0, 2, 3).reshape(Hk, n * block_size, D)[:, :L].float()
        qb = q[b].float().view(Hk, G, D)
        s = torch.matmul(qb, kc.transpose(1, 2).contiguous()) * (D ** -0.5)
        w = torch.softmax(s, dim=-1)
        out[b] = torch.matmul(w, vc).reshape(H, D)
    return out
