"""GPU time per padded document through a nomic-embed-text-shaped encoder whose attention is kernel attention.

The synthetic stand-in for the timing of Experiments/text_transformer/pareto.py:46-65 (encode(): every document
padded to seq_len, CUDA events around the model forward, GPU milliseconds summed over the batches, divided by the
number of documents, pareto.py:101). The LoCo documents and the trained nomic weights need downloads, so the encoder
is NomicBertModel at its default configuration (hidden 768, 12 heads of 64, 12 layers, SwiGLU 3072, rotary) with
max_position_embeddings raised to the sequence length (nomic-embed-text-v1 itself has 8192) and random weights, fed
random token ids. Each document's real length is drawn in [seq_len / 2, seq_len]; the padding
becomes the key mask of every attention layer (inside the sums for the additive kernels, qlka_layer_fwd_masked).
pareto.py's per-sequence RoPE base (an embedding-quality fix) does not change the work and is left out.

    python -m qlka.harness [--kernel add_bump] [--seq_len 8192] [--batch_size 16] [--docs 32] [--layers 12]
                           [--ws_budget_gb 4]

The library's workspace budget (qlka_set_workspace_budget) is set for the run (default 4 GB): every attention call
then runs its B * heads p in chunks whose workspace stays within it, which bounds the model's peak memory.
Prints one JSON line: ms_per_doc, peak_mem_gb and the configuration.
"""

import argparse
import json

import torch

from . import modules


def build_encoder(layers, kernel, device, hidden=768, heads=12, intermediate=3072, seed=0, max_positions=2048):
    """NomicBertModel (SDPA masks) with random weights and every attention layer swapped for `kernel`. The model
    gathers its token-type buffer at the position ids, so it takes at most max_positions tokens."""
    from transformers import NomicBertConfig, NomicBertModel
    torch.manual_seed(seed)
    cfg = NomicBertConfig(num_hidden_layers=layers, hidden_size=hidden, num_attention_heads=heads,
                          intermediate_size=intermediate, max_position_embeddings=max(2048, max_positions))
    model = NomicBertModel._from_config(cfg, attn_implementation="sdpa").to(device).eval()
    return modules.use_kernel_attention(model, kernel)


def synthetic_batches(docs, batch_size, seq_len, vocab, device, seed=0):
    """(input_ids, attention_mask) per batch: random ids, real lengths in [seq_len / 2, seq_len], padded."""
    g = torch.Generator().manual_seed(seed)
    for i in range(0, docs, batch_size):
        b = min(batch_size, docs - i)
        ids = torch.randint(1, vocab, (b, seq_len), generator=g)
        lens = torch.randint(seq_len // 2, seq_len + 1, (b,), generator=g)
        mask = (torch.arange(seq_len)[None, :] < lens[:, None]).long()
        yield (ids * mask).to(device), mask.to(device)


@torch.no_grad()
def encode_time(model, batches):
    """Summed GPU milliseconds of the forwards (pareto.py:58-66) and the pooled embeddings."""
    gpu_ms, pooled = 0.0, []
    for ids, mask in batches:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        hidden = model(input_ids=ids, attention_mask=mask).last_hidden_state
        end.record()
        torch.cuda.synchronize()
        gpu_ms += start.elapsed_time(end)
        m = mask.unsqueeze(-1).to(hidden.dtype)
        pooled.append(torch.nn.functional.normalize((hidden * m).sum(dim=1) / m.sum(dim=1), dim=-1))
    return gpu_ms, torch.cat(pooled)


def run(kernel="add_bump", seq_len=8192, batch_size=16, docs=32, layers=12, device="cuda:0", ws_budget_gb=4.0,
        **model_kw):
    device = torch.device(device)
    from . import _lib
    prev = _lib.load().qlka_set_workspace_budget(int(ws_budget_gb * 1e9))
    try:
        return _run(kernel, seq_len, batch_size, docs, layers, device, ws_budget_gb, **model_kw)
    finally:
        _lib.load().qlka_set_workspace_budget(prev)


def _run(kernel, seq_len, batch_size, docs, layers, device, ws_budget_gb, **model_kw):
    model = build_encoder(layers, kernel, device, max_positions=seq_len, **model_kw)
    if seq_len > model.config.max_position_embeddings:
        raise ValueError(f"seq_len {seq_len} exceeds the encoder's {model.config.max_position_embeddings} positions")
    vocab = model.config.vocab_size
    # one warmup batch at the timed shape (allocator and workspace sizes settle)
    encode_time(model, synthetic_batches(min(docs, batch_size), batch_size, seq_len, vocab, device, seed=1))
    torch.cuda.reset_peak_memory_stats(device)
    gpu_ms, emb = encode_time(model, synthetic_batches(docs, batch_size, seq_len, vocab, device))
    assert torch.isfinite(emb).all(), "non-finite embeddings"
    return {"kernel": kernel, "seq_len": seq_len, "batch_size": batch_size, "num_docs": docs, "layers": layers,
            "hidden": model.config.hidden_size, "heads": model.config.num_attention_heads,
            "ms_per_doc": round(gpu_ms / docs, 3), "gpu_s": round(gpu_ms / 1000, 3),
            "peak_mem_gb": round(torch.cuda.max_memory_allocated(device) / 1e9, 2), "ws_budget_gb": ws_budget_gb,
            "weights": "random (NomicBertConfig defaults)", "data": "synthetic token ids, padded"}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--kernel", default="add_bump", choices=sorted(modules.KERNELS))
    ap.add_argument("--seq_len", type=int, default=8192)
    ap.add_argument("--batch_size", type=int, default=16)
    ap.add_argument("--docs", type=int, default=32)
    ap.add_argument("--layers", type=int, default=12)
    ap.add_argument("--ws_budget_gb", type=float, default=4.0)
    a = ap.parse_args(argv)
    print(json.dumps(run(a.kernel, a.seq_len, a.batch_size, a.docs, a.layers, ws_budget_gb=a.ws_budget_gb)),
          flush=True)


if __name__ == "__main__":
    main()
