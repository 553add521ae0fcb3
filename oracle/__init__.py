"""CPU oracle of the FlashAttention path — TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker. The product (myk_llm_amd) never imports it. See attention.py for what each
function restates and how it is pinned.
"""
