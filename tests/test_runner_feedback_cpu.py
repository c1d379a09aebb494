"""The runner's decode loop with self-feeding decode graphs (llm_runner.c:233-245 schedule), on the CPU:
a fake entry point stands in for the HIP graph. Its decode graphs behave like the real ones (the token
buffer is the `next` buffer and a replay ends with start += 1), and every step's output depends on the
(start, token) the graph actually read, so a stale input after a bucket switch, a skipped write or a
wrong position changes the generated sequence."""

import pytest
import torch

from q4llm import llm_runner


def step_fn(token, start):
    return (token * 31 + start * 7 + 3) % 97


class FakeGraph:
    def __init__(self, C, L, log):
        self.C, self.L, self.log = C, L, log
        self.feeds_back = C == 1
        self.start = torch.zeros(1, dtype=torch.int32)
        self.last = torch.zeros(1, dtype=torch.int32)
        self.next = torch.zeros(1, dtype=torch.int32)
        self.tokens = self.next if self.feeds_back else torch.zeros(C, dtype=torch.int32)

    def replay(self):
        s, t = int(self.start[0]), int(self.tokens[int(self.last[0])])
        self.log.append((self.C, self.L, s, t))
        self.next[0] = step_fn(t, s)
        if self.feeds_back:
            self.start[0] += 1
        return self.next

    def __call__(self, tokens, start, last):
        self.tokens.copy_(torch.as_tensor(tokens, dtype=torch.int32).reshape(-1))
        self.start.fill_(int(start))
        self.last.fill_(int(last))
        return self.replay()

    def set_fed(self, start, token):
        self.start.fill_(int(start))
        self.tokens.fill_(int(token))


class FakeRun:
    """A multi-step decode entry point (LlamaQ4._DecodeRun): `steps` self-feeding steps per replay over
    a ring of token slots, step 0 reading the last slot."""

    def __init__(self, L, steps, log):
        self.C, self.L, self.steps, self.log = 1, L, steps, log
        self.feeds_back = True
        self.start = torch.zeros(1, dtype=torch.int32)
        self.ring = torch.zeros(steps, dtype=torch.int32)

    def replay(self):
        for i in range(self.steps):
            s, t = int(self.start[0]), int(self.ring[(i - 1) % self.steps])
            self.log.append((1, self.L, s, t))
            self.ring[i] = step_fn(t, s)
            self.start[0] += 1
        return self.ring

    def set_fed(self, start, token):
        self.start.fill_(int(start))
        self.ring[self.steps - 1] = int(token)


class FakeModel:
    device = torch.device("cpu")
    max_ctx = 64

    def __init__(self):
        self.graphs, self.log = {}, []

    def new_caches(self):
        return []

    def entry_point(self, C, L, caches, steps=1):
        if (C, L, steps) not in self.graphs:
            self.graphs[(C, L, steps)] = FakeGraph(C, L, self.log) if steps == 1 else FakeRun(L, steps, self.log)
        return self.graphs[(C, L, steps)]


def expected(prompt, max_new, chunk, buckets):
    """The same recurrence with explicit inputs at every step."""
    n = len(prompt)
    last_chunk = prompt[(n - 1) // chunk * chunk:]
    nxt = step_fn(last_chunk[-1], (n - 1) // chunk * chunk)
    out, pos = [nxt], n
    while len(out) < max_new and llm_runner.pick_bucket(buckets, pos + 1) > 0:
        out.append(step_fn(out[-1], pos))
        pos += 1
    return out


@pytest.mark.parametrize("decode_steps", [1, 8, 5])
def test_decode_feedback_across_bucket_switches(monkeypatch, decode_steps):
    """One-step replays, and multi-step replays mixed with single steps near the bucket switches and
    the end of the generation."""
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    model = FakeModel()
    prompt = [5, 9, 2, 44, 17, 8, 60, 1, 3, 12]
    buckets = [16, 32, 64]
    res = llm_runner.run(model, prompt, max_new_tokens=40, chunk=8, buckets=buckets, warmup=1,
                         decode_steps=decode_steps)
    assert res["tokens"] == expected(prompt, 40, 8, buckets)
    # decode steps read (start, token) = (pos, previous token) on every bucket, including right after
    # the switches at positions 16 and 32
    dec = [(L, s, t) for (C, L, s, t) in model.log if C == 1 and s >= len(prompt)]
    toks = res["tokens"]
    assert [(s, t) for _, s, t in dec[-(len(toks) - 1):]] == [(len(prompt) + i, toks[i]) for i in range(len(toks) - 1)]
    assert {L for L, _, _ in dec} == {16, 32, 64}


def test_multi_step_decode_runs_are_used_and_stop_ids_truncate(monkeypatch):
    """With 8 steps per replay the run takes multi-step replays inside each bucket, and a stop id met
    inside a replay ends the generation at that token (the tokens match the one-step runner's)."""
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)
    prompt = [5, 9, 2, 44, 17, 8, 60, 1, 3, 12]
    buckets = [16, 32, 64]
    ref = llm_runner.run(FakeModel(), prompt, max_new_tokens=45, chunk=8, buckets=buckets, decode_steps=1)["tokens"]
    model = FakeModel()
    res = llm_runner.run(model, prompt, max_new_tokens=45, chunk=8, buckets=buckets, decode_steps=8)
    assert res["tokens"] == ref
    assert any(isinstance(g, FakeRun) for g in model.graphs.values())
    stop = ref[20]
    first = ref.index(stop)
    for k in (1, 8):
        got = llm_runner.run(FakeModel(), prompt, max_new_tokens=45, chunk=8, buckets=buckets, stop_ids=(stop,),
                             decode_steps=k)["tokens"]
        assert got == ref[:first + 1], k
