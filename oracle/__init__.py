"""CPU oracle for the AIOS-IME paged attention path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference (7155/aios) computes on
the attention-backend hot path, so that the gfx950 HIP kernels can be checked
against it.  It is imported only by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``; the product package
``aios_amd`` never imports it and has no CPU fallback.

Modules and what pins each function (the checks live in tests/test_oracle.py):

  kv_store.py   paged KV scatter (kernel/store.py:8-61)
                pinned by the reference's scatter known answer
                (resources/lesson-30-triton-kv-store/run_lesson30.py:7-23) and
                by brute-force index_put on random inputs.
  metadata.py   cu_seqlens / flat page indices / last-token rows
                (attention/flashinfer.py:209-250)
                pinned by resources/lesson-26-flashinfer-backend/run_lesson26.py
                and resources/lesson-32-flashinfer-paged-attention/run_lesson32.py
                known answers.
  attention.py  offset-causal GQA paged attention in float64
                (attention/flashinfer.py:33-91, 328-372, 374-394) pinned by
                torch's scaled_dot_product_attention (an independent library
                routine), by the reference's own test case
                (tests/test_attention_backend.py:25-53: seed 17, cached_len in
                {0, 2}), and by closed forms (constant keys -> mean of visible
                values; one visible key -> that value; permutation of pages).
                The log-sum-exp merge is pinned by the online-softmax known
                answer (resources/lesson-41-flashattention-online-softmax/
                run_lesson41.py) and by split-anywhere == unsplit.
  sdpa_cpu.py   line-for-line torch restatement of the reference's CPU
                attention path (_sdpa_prefill_attention, flashinfer.py:33-91
                and the per-request loop :328-372); used as the CPU baseline.
                Pinned against attention.py.
  prefix.py     token-LCP prefix-reuse plan (ime.py:1116-1168), pinned by the
                four cases of resources/lesson-14-prefix-kv-reuse/run_lesson14.py.
  attnres.py    Block-AttnRes depth mixer in float64 (kernel/attnres.py:8-127,
                models/minimind_ime.py:27-74, 92-190): the expanded (production)
                form and the materialised form, pinned against each other,
                against the reference's zero-query known answer
                (tests/test_ime_attnres.py:59-66), a hand-computed two-source
                case, closed forms (one source, identical sources, scale
                invariance of the RMS score), and its bf16 rounding against
                torch's conversion.
  model.py      float32 CPU restatement of the Qwen3 decoder and the greedy
                CandidateGroup decode loop (models/qwen3.py:31-173,
                layers/*.py, ime.py:891-1251) used for full-model Top-1/3
                parity.  The standard Qwen3 trunk is pinned against an
                independent implementation, transformers' Qwen3ForCausalLM
                (tests/test_oracle_hf.py: the same weights through the
                exported bundle's HF tensor names; logits equal within 1e-5
                at G = 4 / D = 96, G = 2 / D = 128 and an untied G = 3 /
                D = 64 head, greedy candidates token for token), and by
                closed forms (RoPE pair rotation by pos * theta^(-2i/D),
                identity at position 0, norm preservation; with every
                projection zeroed the logits are RMSNorm(embed) @ embed^T).
                The Block-AttnRes trunk composition is pinned by its
                zero-query closed form (every depth softmax uniform, so the
                trunk at eps 1e-12 equals transformers' Qwen3 on the same
                weights, at 8 layers in 4 blocks and 6 layers in 2 blocks;
                a planted stale-source MLP mixer fails it by more than
                1e-2); non-zero queries by the mixer's own known answers.
  cpu_decoder.py  KV-cached CPU decoder over the paged pool (the same
                forward, attention by sdpa_cpu.py), bf16 or fp32: the
                full-model leg of bench.py's CPU baseline.  Pinned against
                model.py (float32: prefix prefill, LCP extension and decode
                steps over scattered pages equal the dense recomputation's
                logits within 1e-4; a page relabelling changes nothing).
"""
