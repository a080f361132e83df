"""The enqueue entry points under HIP graph capture (torch.cuda.graph): a decode step of a small model - the
batched append of a token's keys and values to every layer's cache (pitch_enqueue_encode_batch) and the
allocation-free attention of every layer (pitch_enqueue_attention_decode_noalloc) - captured once and replayed
for several tokens. The library's enqueue paths issue only kernel launches (no memset, copy, allocation or
synchronisation), so a replay must write exactly what the same calls write eagerly: each replay is checked bit
for bit against eager calls on the same inputs, with the program's own eager work and synchronisations between
the replays.
"""
import pytest

pytestmark = pytest.mark.gpu


def test_decode_step_graph_replays_match_eager(q):
    import torch
    import pitch_amd as P
    dev = q.device
    layers, heads, nq, d, T = 4, 4, 2, 128, 700
    kcfg, vcfg = P.QuantConfig("turboQuant", d, 4, 11), P.QuantConfig("turboQuant", d, 3, 12)
    g = torch.Generator(device=dev).manual_seed(21)

    def caches():
        out = []
        for _ in range(layers):
            kc = torch.zeros(T * heads * kcfg.codeStride, dtype=torch.uint8, device=dev)
            vc = torch.zeros(T * heads * vcfg.codeStride, dtype=torch.uint8, device=dev)
            ks, vs = torch.zeros(T * heads, device=dev), torch.zeros(T * heads, device=dev)
            out.append((kc, ks, vc, vs))
        return out

    # a prefix of T - 8 tokens, encoded eagerly into both sets of caches
    prefix = T - 8
    Kp = [torch.randn(prefix * heads, d, generator=g, device=dev) for _ in range(layers)]
    Vp = [torch.randn(prefix * heads, d, generator=g, device=dev) for _ in range(layers)]
    eager, graphed = caches(), caches()
    for c in (eager, graphed):
        for l in range(layers):
            q.enqueueEncode(Kp[l], c[l][0], c[l][1], prefix * heads, kcfg)
            q.enqueueEncode(Vp[l], c[l][2], c[l][3], prefix * heads, vcfg)
    # the step's inputs and outputs live in fixed buffers that the graph reads and writes
    new_k = [torch.zeros(heads, d, device=dev) for _ in range(layers)]
    new_v = [torch.zeros(heads, d, device=dev) for _ in range(layers)]
    Q = [torch.zeros(heads, nq, d, device=dev) for _ in range(layers)]
    out_g = [torch.zeros(heads, nq, d, device=dev) for _ in range(layers)]

    def step(c, outs, t, kt, vt):
        kb, vb = kt, vt
        kb.enqueue(heads, codesOffsets=t * heads * kcfg.codeStride, scalesOffsets=t * heads * 4)
        vb.enqueue(heads, codesOffsets=t * heads * vcfg.codeStride, scalesOffsets=t * heads * 4)
        for l in range(layers):
            q.enqueueAttentionDecode(Q[l], c[l][0], c[l][1], c[l][2], c[l][3], outs[l], t + 1, kcfg, vcfg,
                                     qPerKv=nq, kvHeads=heads, tokenStride=heads, headStride=1, noAlloc=True)

    tabs = {}
    for name, c in (("eager", eager), ("graph", graphed)):
        tabs[name] = (P.EncodeBatch(q, kcfg, new_k, [x[0] for x in c], [x[1] for x in c]),
                      P.EncodeBatch(q, vcfg, new_v, [x[2] for x in c], [x[3] for x in c]))
    # one eager call first: the library resolves its per-device scratch address outside the capture
    warm = torch.zeros(heads, nq, d, device=dev)
    q.enqueueAttentionDecode(Q[0], eager[0][0], eager[0][1], eager[0][2], eager[0][3], warm, prefix, kcfg, vcfg,
                             qPerKv=nq, kvHeads=heads, tokenStride=heads, headStride=1, noAlloc=True)
    torch.cuda.synchronize()
    # capture one step per token position (offsets are fixed in a captured graph)
    graphs = []
    stream = torch.cuda.Stream()
    for t in range(prefix, T):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=stream):
            step(graphed, out_g, t, *tabs["graph"])
        graphs.append(gr)
    torch.cuda.synchronize()
    out_e = [torch.zeros_like(o) for o in out_g]
    for i, t in enumerate(range(prefix, T)):
        # new inputs for this token, written in place
        for l in range(layers):
            new_k[l].copy_(torch.randn(heads, d, generator=g, device=dev))
            new_v[l].copy_(torch.randn(heads, d, generator=g, device=dev))
            Q[l].copy_(torch.randn(heads, nq, d, generator=g, device=dev))
        torch.cuda.synchronize()
        graphs[i].replay()
        torch.cuda.synchronize()
        step(eager, out_e, t, *tabs["eager"])
        torch.cuda.synchronize()
        for l in range(layers):
            assert torch.equal(out_g[l], out_e[l]), f"token {t} layer {l}: attention output differs"
            for a, b in zip(graphed[l], eager[l]):
                assert torch.equal(a, b), f"token {t} layer {l}: cache differs"
        # eager work of the program between replays
        _ = (torch.randn(1024, device=dev) * 2).sum().item()
    # the captured steps replayed again (the last one), once more after eager work: same bytes
    graphs[-1].replay()
    torch.cuda.synchronize()
    for l in range(layers):
        assert torch.equal(out_g[l], out_e[l])
