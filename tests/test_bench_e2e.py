"""The E2E benchmark's workload (nanovllm.bench_e2e.make_workload): the
reference benchmark's convention, prompt and output lengths uniform in
[100, max] (the lower bound shrinks with a smaller max), seeded."""
from nanovllm.bench_e2e import make_workload


def test_workload_lengths_and_seed():
    prompts, params = make_workload(64, 1024, 1024, seed=0)
    assert all(100 <= len(p) <= 1024 for p in prompts)
    assert all(100 <= sp.max_tokens <= 1024 and sp.ignore_eos and sp.temperature == 0.0 for sp in params)
    assert all(0 <= t <= 10000 for p in prompts for t in p)
    again, _ = make_workload(64, 1024, 1024, seed=0)
    assert again == prompts
    short, sparams = make_workload(8, 24, 4, seed=1)
    assert all(1 <= len(p) <= 24 for p in short) and all(1 <= sp.max_tokens <= 4 for sp in sparams)
