"""A forward replayed from a HIP graph, for callers with static input buffers
(serving loops, fixed-shape batches).

A forward of several short kernels costs host work around them (cache-key
walks over the parameters, argument marshalling, output allocation) that can
take as long as the kernels themselves; captured once, each call is one
graph launch. The graph keeps the tensors it was captured
on: each call writes its batch into the captured inputs (or passes them
unchanged) and reads the captured output, which the next call overwrites.
The parameters must not be replaced or modified after capture (the derived
tables the graph reads were built for them); capture again after a change.
"""
import torch


class CapturedForward:
    """``fn(*inputs)`` captured into a graph. ``inputs`` are device tensors
    the caller keeps (the graph reads them at these addresses)."""

    def __init__(self, fn, *inputs, warmup=2):
        if not inputs or any(not torch.is_tensor(t) or t.device.type != "cuda" for t in inputs):
            raise ValueError("CapturedForward: inputs must be device tensors")
        self.fn, self.inputs = fn, inputs
        # build every cached table (hard codes, placements, plans, launch
        # sequences keyed by stream) outside the capture, on the stream the
        # capture then uses, so the capture records launches and builds nothing
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.no_grad(), torch.cuda.stream(side):
            for _ in range(warmup):
                fn(*inputs)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph, stream=side):
            self.output = fn(*inputs)

    def __call__(self, *batch):
        """Replay on ``batch`` (copied into the captured inputs unless it is
        them) and return the captured output tensor."""
        if batch:
            if len(batch) != len(self.inputs):
                raise ValueError("CapturedForward: %d inputs captured, %d given"
                                 % (len(self.inputs), len(batch)))
            for dst, src in zip(self.inputs, batch):
                if src is not dst:
                    dst.copy_(src)
        self.graph.replay()
        return self.output
