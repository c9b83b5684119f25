"""The mia-serve line protocol on the GPU engine (motoria_amd/mia-serve,
host/server.c), driven over pipes as the reference's engine package drives
it (tools/internal/engine/protocol.go:1-13), on the tiny model with the
serve test's chat vocabulary (tools/e2e/serve_test.go:16-47). Besides the
reference's own serve checks (context kept across turns, only the new turn
prefilled, RESET, context_full with the engine still usable), every
generated token is compared with the oracle's model step and sampler run
over the same conversation, including the sampler state carried from turn
to turn, and SIGUSR1 cancels a prefill and rolls the context back."""
import ctypes
import os
import signal
import subprocess
import sys

import numpy as np
import pytest

import motoria_amd as M
import mia_writer as MW

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


class Serve:
    def __init__(self, path, ctx, seed=1):
        self.p = subprocess.Popen([M.SERVE_PATH, "-m", path, "--ram", "64M", "-c", str(ctx),
                                   "--seed", str(seed)], stdin=subprocess.PIPE,
                                  stdout=subprocess.PIPE, stderr=subprocess.PIPE)
        line = self.line()
        assert line.startswith("READY "), line
        self.info = dict(kv.split("=") for kv in line.split()[1:])

    def line(self):
        raw = self.p.stdout.readline()
        if not raw:
            raise RuntimeError("mia-serve ended: " + self.p.stderr.read().decode())
        return raw.decode().rstrip("\n")

    def send(self, data):
        self.p.stdin.write(data)
        self.p.stdin.flush()

    def chat(self, text, max_tokens, t=0.0, p=1.0, think=0, on_prog=None):
        """(events, done dict or None, error (code, msg) or None); events are
        ("PROG", done, total) and ("TOK", bytes)."""
        raw = text.encode()
        self.send(b"CHAT %d %d %g %g %d\n" % (len(raw), max_tokens, t, p, think) + raw)
        events = []
        while True:
            line = self.line()
            head = line.split(" ", 1)[0]
            if head == "PROG":
                _, a, b = line.split()
                events.append(("PROG", int(a), int(b)))
                if on_prog:
                    on_prog(int(a))
            elif head == "TOK":
                n = int(line.split()[1])
                events.append(("TOK", self.p.stdout.read(n)))
            elif head == "DONE":
                return events, dict(kv.split("=") for kv in line.split()[1:]), None
            elif head == "ERR":
                _, code, msg = line.split(" ", 2)
                return events, None, (code, msg)
            else:
                raise AssertionError("unexpected line " + line)

    def close(self):
        try:
            self.send(b"QUIT\n")
            self.p.wait(timeout=60)
        finally:
            if self.p.poll() is None:
                self.p.kill()
                self.p.wait()


class Reference:
    """The conversation as the reference's serve loop runs it
    (src/app/serve.c:64-143), on the oracle's model step and sampler."""

    def __init__(self, oracle, path, ctx, seed):
        self.O, self.ctx = oracle, ctx
        self.fm = MW.FileModel(oracle, path, MW.TINY)
        self.kc, self.vc = self.fm.kv_cache(ctx)
        self.tok = M.Bpe(MW.chat_tokenizer())
        self.s = oracle.Sampler()
        oracle.lib().orc_sampler_init(ctypes.byref(self.s), 0.7, 0.8, MW.TINY["vocab"], seed)
        self.pos = 0

    def step(self, tok):
        lg, _ = self.O.model_step(self.fm.model, self.kc, self.vc, self.ctx, tok, self.pos,
                                  nthreads=4)
        self.pos += 1
        return lg

    def chat(self, text, max_tokens, t=0.0, p=1.0, think=0):
        self.s.temperature = t
        self.s.top_p = p if 0.0 < p <= 1.0 else 1.0
        ids = self.tok.encode(M.chat_turn_text(text, think, self.pos > 0))
        for i in ids:
            lg = self.step(i)
        out, reason = [], "length"
        while len(out) < max_tokens:
            if self.pos >= self.ctx:
                reason = "ctx"
                break
            nxt = self.O.lib().orc_sample(ctypes.byref(self.s), lg.ctypes.data)
            if self.tok.is_stop(nxt):
                reason = "stop"
                break
            out.append(self.tok.piece(nxt))
            lg = self.step(nxt)
        return len(ids), out, reason


@pytest.fixture(scope="module")
def chat_model(oracle, tmp_path_factory):
    path = str(tmp_path_factory.mktemp("serve") / "chat.mia")
    MW.synthetic(oracle, path, MW.TINY, MW.Q8_0, 5, tokenizer=MW.chat_tokenizer())
    return path


def tokens(events):
    return [e[1] for e in events if e[0] == "TOK"]


def progress(events):
    return [e for e in events if e[0] == "PROG"]


def test_serve_keeps_context_across_turns(oracle, chat_model):
    say("test_serve_keeps_context_across_turns")
    s = Serve(chat_model, 512)
    ref = Reference(oracle, chat_model, 512, 1)
    try:
        assert s.info["layers"] == "2" and s.info["experts"] == "8" and s.info["ctx"] == "512"
        assert s.info["active"] == "2" and s.info["wtype"] == "q8_0"
        ev, first, err = s.chat("hi", 4)
        assert err is None
        n, want, reason = ref.chat("hi", 4)
        assert int(first["prompt"]) == n == len(progress(ev))
        assert progress(ev)[-1] == ("PROG", n, n)
        assert tokens(ev) == want and int(first["gen"]) == len(want) <= 4
        assert first["reason"] == reason and reason in ("length", "stop")
        ev, second, err = s.chat("ok", 4)
        n2, want2, _ = ref.chat("ok", 4)
        assert err is None and tokens(ev) == want2
        assert int(second["ctx_used"]) > int(first["ctx_used"])
        assert int(second["prompt"]) == n2 < int(second["ctx_used"])  # only the new turn
        s.send(b"RESET\n")
        assert s.line() == "OK"
        ev, again, err = s.chat("hi", 4)
        assert err is None and again["ctx_used"] == first["ctx_used"]
        assert tokens(ev) == want
        say("  turns: %s / %s tokens, ctx %s -> %s" % (first["gen"], second["gen"],
                                                       first["ctx_used"], second["ctx_used"]))
    finally:
        s.close()


@pytest.mark.parametrize("t,p", [(0.8, 0.9), (1.2, 1.0)])
def test_serve_sampling_matches_reference(oracle, chat_model, t, p):
    say("test_serve_sampling_matches_reference T=%g top_p=%g" % (t, p))
    s = Serve(chat_model, 256, seed=7)
    ref = Reference(oracle, chat_model, 256, 7)
    try:
        for text in ("tell me", "more", "and again"):
            ev, done, err = s.chat(text, 12, t, p)
            n, want, reason = ref.chat(text, 12, t, p)
            assert err is None and tokens(ev) == want and done["reason"] == reason, text
    finally:
        s.close()


def test_serve_context_limits_and_bad_requests(oracle, chat_model):
    say("test_serve_context_limits_and_bad_requests")
    s = Serve(chat_model, 48)
    try:
        ev, done, err = s.chat("a" * 200, 4)
        assert done is None and err[0] == "context_full" and not ev
        ev, done, err = s.chat("hi", 2)  # still usable
        assert err is None and done["reason"] in ("length", "stop")
        # generation runs into the end of the context
        s.send(b"RESET\n")
        assert s.line() == "OK"
        ev, done, err = s.chat("x" * 4, 100)
        assert err is None and done["reason"] in ("ctx", "stop")
        if done["reason"] == "ctx":
            assert done["ctx_used"] == "48"
        s.send(b"FLY\n")
        assert s.line().startswith("ERR bad_request unknown command")
        s.send(b"CHAT -5 4 0 1 0\n")
        assert s.line().startswith("ERR bad_request")
    finally:
        s.close()


def test_serve_cancel_rolls_back(oracle, chat_model):
    """SIGUSR1 after the first PROG line: the CHAT ends with reason=cancel
    and, when that happened during the prefill, the context is rolled back;
    the next turn is then the fresh conversation's."""
    say("test_serve_cancel_rolls_back")
    s = Serve(chat_model, 1024)
    try:
        _, fresh, _ = s.chat("hi", 3)
        s.send(b"RESET\n")
        assert s.line() == "OK"
        sent = []

        def cancel(done):
            if not sent:
                s.p.send_signal(signal.SIGUSR1)
                sent.append(done)

        text = "z" * 600
        n = len(M.Bpe(MW.chat_tokenizer()).encode(M.chat_turn_text(text, 0, 0)))
        ev, done, err = s.chat(text, 3, on_prog=cancel)
        assert err is None and done["reason"] == "cancel"
        if int(done["prompt"]) < n:  # cancelled in the prefill
            assert done["gen"] == "0" and int(done["prompt"]) == len(progress(ev))
            assert done["ctx_used"] == "0"  # rolled back to the turn's start
            ev, again, _ = s.chat("hi", 3)
            assert again["ctx_used"] == fresh["ctx_used"]
        say("  cancelled after %s of the prompt's tokens" % done["prompt"])
    finally:
        s.close()
