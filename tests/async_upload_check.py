"""Helper of tests/test_gpu_pjrt.py::test_upload_does_not_wait_for_queued_kernels,
run as its own process so that the plugin's two streams are the only HIP
streams in it, as in a JAX process (HIP maps a process's streams onto at most
GPU_MAX_HW_QUEUES hardware queues, so after other libraries have made
streams the transfer stream can share a hardware queue with the compute
stream, and then a copy queued behind kernels waits for them).

Queues about 26 ms of attention, uploads a small buffer, and checks that its
ready event completes while the attention is still running and that a
program queued after the upload reads its bytes.  Then the reuse case: with
attention reading buffer A queued, A is destroyed and a buffer B of the same
size is uploaded (the pool hands B A's block); every queued attention must
still see A's bytes and B must hold its own.  Prints one line per trial;
exits non-zero on failure."""

import os
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mccl-jax_amd")]

import numpy as np  # noqa: E402

from mi355x_pjrt import modules, pjrt  # noqa: E402
from oracle import bf16, inputs  # noqa: E402


def main():
    p = pjrt.Plugin()
    client = p.client()
    d = inputs.c3_sdpa(8192)
    e = client.compile(modules.sdpa(4, 16, 8192, 128, True))
    red = client.compile(modules.reduce_sum(4, 8))
    bufs = [client.put(d[k], pjrt.BF16) for k in ("q", "k", "v")]
    for b in bufs:
        b.ready()
    x = (np.arange(4 * 8, dtype=np.float32).reshape(4, 8) % 7).astype(np.float32)
    for trial in range(3):
        outs, ev = [], None
        for _ in range(24):
            if ev is not None:
                p.call("Event_Destroy", event=ev)
            o, ev = e.execute(bufs, wait="event")
            outs += o
        t0 = time.perf_counter()
        xb = client.put(bf16.to_bf16_bits(x), pjrt.BF16)  # small integers: exact in bf16
        t1 = time.perf_counter()
        xb.ready()
        t2 = time.perf_counter()
        busy = not p.event_ready(ev)
        (y,) = red.execute([xb])
        got = y.to_numpy()
        p.await_event(ev)
        print(f"trial {trial}: put {1e3 * (t1 - t0):.3f} ms, upload ready {1e3 * (t2 - t1):.3f} ms later, "
              f"attention still running then: {busy}", flush=True)
        if not busy:
            print("FAIL: the upload waited for the queued kernels", flush=True)
            return 1
        if not np.array_equal(got, x.sum(-1)):
            print(f"FAIL: program after the upload read {got}", flush=True)
            return 1
        for b in outs + [xb, y]:
            b.destroy()
    return check_reuse(p, client, e, bufs, d)


def check_reuse(p, client, e, bufs, d):
    (want,) = e.execute(bufs)
    want_np = want.to_numpy()
    want.destroy()
    other = bf16.to_bf16_bits(-bf16.from_bf16_bits(d["q"]))  # same size, different bytes
    for trial in range(2):
        a = client.put(d["q"], pjrt.BF16)
        a.ready()
        outs, ev = [], None
        for _ in range(24):
            if ev is not None:
                p.call("Event_Destroy", event=ev)
            o, ev = e.execute([a, bufs[1], bufs[2]], wait="event")
            outs += o
        where = a.device_pointer
        a.destroy()
        b = client.put(other, pjrt.BF16)
        reused = b.device_pointer == where
        busy = not p.event_ready(ev)
        p.await_event(ev)
        bad = [i for i, o in enumerate(outs) if not np.array_equal(o.to_numpy(), want_np)]
        b_ok = np.array_equal(b.to_numpy(), other)
        print(f"reuse trial {trial}: block reused {reused}, attention still running at upload {busy}, "
              f"outputs changed {len(bad)}/{len(outs)}, B intact {b_ok}", flush=True)
        if bad or not b_ok:
            print("FAIL: an upload into a reused block raced the kernels reading it", flush=True)
            return 1
        for x in outs + [b]:
            x.destroy()
    return 0


if __name__ == "__main__":
    sys.exit(main())
