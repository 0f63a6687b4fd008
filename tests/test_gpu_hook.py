"""The transformers attention hook end to end: a small random-weight Qwen2 CausalLM runs
prefill and greedy decode steps through the device page pool, the append kernel and the
decode/prefill wrappers (the flow of ecahlang/main.py:424-470, 320-347), and every step's
logits are checked against the same model with transformers' own SDPA attention over the
full token sequence (no cache)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _model(dtype=torch.float16):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(0)
    cfg = Qwen2Config(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=2048,
                      initializer_range=0.2)
    return Qwen2ForCausalLM(cfg).to(DEV, dtype).eval()


def _set_impl(model, name):
    if hasattr(model, "set_attn_implementation"):
        model.set_attn_implementation(name)
    else:
        model.config._attn_implementation = name


def _close(got, ref, what):
    got, ref = got.float().cpu().numpy(), ref.float().cpu().numpy()
    err = np.abs(got - ref).max() / max(np.abs(ref).max(), 1e-6)
    assert err < 2e-2, f"{what}: relative max error {err:.3g}"


@torch.no_grad()
@pytest.mark.parametrize("model_dtype", [torch.float16, torch.float32])
def test_hook_prefill_and_decode_match_sdpa_model(model_dtype):
    """fp16 model over an fp16 cache; and an fp32 model over the fp16 cache, where the hook
    casts q/k/v to the cache's dtype and the output back (main.py:50-53, 95-96)."""
    from ecahlang_amd import hook
    from ecahlang_amd.manager import AutoKVCacheManager
    from ecahlang_amd.wrappers import BatchDecodeWithPagedKVCacheWrapper, BatchPrefillWithPagedKVCacheWrapper

    hook.register()
    model = _model(model_dtype)
    L, hkv, hq, d = 2, 2, 4, 64
    mgr = AutoKVCacheManager(L, hkv, d, vocab_size=512, dtype=torch.float16, device=DEV,
                             total_gpu_mem_bytes=300 * 16 * hkv * d * 2 * 2 * L, mem_utilization=1.0)
    gen = torch.Generator().manual_seed(5)
    lens = [5, 17, 9, 32]
    ids = [f"req{i}" for i in range(len(lens))]
    seqs = [torch.randint(0, 512, (n,), generator=gen).tolist() for n in lens]

    def reference_last_logits():
        _set_impl(model, "sdpa")
        out = []
        for s in seqs:
            x = torch.tensor(s, device=DEV)[None]
            out.append(model(input_ids=x, use_cache=False).logits[0, -1])
        return torch.stack(out)

    # ---- prefill: all prompts in one ragged batch (main.py:424-458)
    for rid, n in zip(ids, lens):
        mgr.allocate(rid, n)
    append_indptr = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    mgr.prepare_append_metadata(ids, append_indptr)
    pw = BatchPrefillWithPagedKVCacheWrapper(torch.empty(32 << 20, dtype=torch.uint8, device=DEV), "NHD")
    pw.plan(append_indptr, mgr._cached_kv_indptr, mgr._cached_kv_indices, mgr._cached_kv_last_page_len,
            hq, hkv, d, mgr.block_size, causal=True, q_data_type=torch.float16)
    mgr.prefill_layer_idx = 0
    input_ids = torch.tensor(sum(seqs, []), device=DEV)[None]
    position_ids = torch.cat([torch.arange(n) for n in lens]).to(DEV)[None]
    _set_impl(model, hook.HOOK_NAME)
    logits = model(input_ids=input_ids, position_ids=position_ids, use_cache=False, wrapper=pw, manager=mgr,
                   prefill=True, append_indptr=append_indptr).logits[0]
    assert mgr.prefill_layer_idx == L
    ref = reference_last_logits()
    _close(logits[append_indptr[1:].long() - 1], ref, "prefill")

    # ---- decode steps (main.py:320-347 without the graph): one token per sequence
    dw = BatchDecodeWithPagedKVCacheWrapper(torch.empty(32 << 20, dtype=torch.uint8, device=DEV), "NHD")
    for step in range(4):
        nxt = ref.argmax(-1).tolist()
        pos = [len(s) for s in seqs]
        for rid, s, t in zip(ids, seqs, nxt):
            s.append(t)
            mgr.append_tokens(rid, 1)
        step_indptr = torch.arange(len(ids) + 1, dtype=torch.int32, device=DEV)
        mgr.prepare_append_metadata(ids, step_indptr)
        dw.plan(mgr._cached_kv_indptr, mgr._cached_kv_indices, mgr._cached_kv_last_page_len, hq, hkv, d,
                mgr.block_size, pos_encoding_mode="NONE", q_data_type=torch.float16)
        mgr.decode_layer_idx = 0
        _set_impl(model, hook.HOOK_NAME)
        logits = model(input_ids=torch.tensor(nxt, device=DEV)[None], position_ids=torch.tensor(pos, device=DEV)[None],
                       use_cache=False, wrapper=dw, manager=mgr, prefill=False, append_indptr=step_indptr).logits[0]
        assert mgr.decode_layer_idx == L
        ref = reference_last_logits()
        _close(logits, ref, f"decode step {step}")
    assert mgr.pool_errors() == 0


@torch.no_grad()
def test_hook_graph_captured_decode_with_padding_bucket():
    """main.py:130-157, 320-381: one decode step captured in a graph at bucket 8 for 5 real
    sequences (3 padding rows on the padding pages), re-planned and replayed per step."""
    from ecahlang_amd import hook
    from ecahlang_amd.manager import AutoKVCacheManager
    from ecahlang_amd.wrappers import BatchDecodeWithPagedKVCacheWrapper, BatchPrefillWithPagedKVCacheWrapper

    hook.register()
    model = _model()
    L, hkv, hq, d = 2, 2, 4, 64
    mgr = AutoKVCacheManager(L, hkv, d, vocab_size=512, dtype=torch.float16, device=DEV,
                             total_gpu_mem_bytes=400 * 16 * hkv * d * 2 * 2 * L, mem_utilization=1.0)
    mgr.init_cuda_graph_buffers([1, 2, 4, 8])
    gen = torch.Generator().manual_seed(9)
    lens = [3, 16, 31, 40, 12]
    ids = [f"g{i}" for i in range(len(lens))]
    seqs = [torch.randint(0, 512, (n,), generator=gen).tolist() for n in lens]
    B, bucket = len(ids), 8

    def reference_last_logits():
        _set_impl(model, "sdpa")
        return torch.stack([model(input_ids=torch.tensor(s, device=DEV)[None], use_cache=False).logits[0, -1]
                            for s in seqs])

    # prefill, eager
    for rid, n in zip(ids, lens):
        mgr.allocate(rid, n)
    append_indptr = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    mgr.prepare_append_metadata(ids, append_indptr)
    pw = BatchPrefillWithPagedKVCacheWrapper(torch.empty(32 << 20, dtype=torch.uint8, device=DEV), "NHD")
    pw.plan(append_indptr, mgr._cached_kv_indptr, mgr._cached_kv_indices, mgr._cached_kv_last_page_len,
            hq, hkv, d, 16, causal=True, q_data_type=torch.float16)
    mgr.prefill_layer_idx = 0
    _set_impl(model, hook.HOOK_NAME)
    model(input_ids=torch.tensor(sum(seqs, []), device=DEV)[None],
          position_ids=torch.cat([torch.arange(n) for n in lens]).to(DEV)[None], use_cache=False,
          wrapper=pw, manager=mgr, prefill=True, append_indptr=append_indptr)
    ref = reference_last_logits()

    dw = BatchDecodeWithPagedKVCacheWrapper(torch.empty(32 << 20, dtype=torch.uint8, device=DEV), "NHD")
    static_ids = torch.zeros(1, bucket, dtype=torch.long, device=DEV)
    static_pos = torch.zeros(1, bucket, dtype=torch.long, device=DEV)

    def step_fn():
        mgr.decode_layer_idx = 0
        return model(input_ids=static_ids, position_ids=static_pos, use_cache=False, wrapper=dw, manager=mgr,
                     prefill=False, append_indptr=mgr._cg_append_indptr[bucket]).logits[0]

    graph, out = None, None
    capture_stream = torch.cuda.Stream()
    for step in range(5):
        nxt = ref.argmax(-1).tolist()
        pos = [len(s) for s in seqs]
        for rid, s, t in zip(ids, seqs, nxt):
            s.append(t)
            mgr.append_tokens(rid, 1)
        mgr.fill_cuda_graph_metadata(bucket, ids)
        dw.plan(mgr._cg_kv_indptr[bucket], mgr._cg_kv_indices[bucket], mgr._cg_kv_last_page_len[bucket],
                hq, hkv, d, 16, pos_encoding_mode="NONE", q_data_type=torch.float16)
        static_ids.zero_()
        static_pos.zero_()
        static_ids[0, :B] = torch.tensor(nxt, device=DEV)
        static_pos[0, :B] = torch.tensor(pos, device=DEV)
        _set_impl(model, hook.HOOK_NAME)
        mgr.cuda_graph_mode = True
        if graph is None:
            with torch.cuda.stream(capture_stream):
                for _ in range(2):  # warm-up, as CUDAGraphDecodeWrapper.warmup
                    step_fn()
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=capture_stream):
                    out = step_fn()
        graph.replay()
        torch.cuda.synchronize()
        mgr.cuda_graph_mode = False
        logits = out[:B].clone()
        ref = reference_last_logits()
        _close(logits, ref, f"graph decode step {step}")
    assert mgr.pool_errors() == 0
