"""GPU token sampler for the serving loop, on the vkwr_sampling kernels.

A ``GpuSampler`` turns a step's logits [S, V] (fp16 or fp32) into S tokens with
temperature / top-k / top-p sampling (the semantics of the reference's
temperature_topk_topp, csrc/sampling/sampling.cu:438-646, 842-915).  Row r of a
call draws from Philox subsequence r of the sampler's seed; every call advances
the counters of the rows it used.  Buffers (states, fp32 logits, tokens, and
the probability scratch of vocabularies above 65536) are allocated once for
``max_rows`` rows, so a call allocates nothing.
"""
import torch

from vkwr_amd import capi


class GpuSampler:
    def __init__(self, max_rows, vocab, device, seed=0, temperature=1.0, top_k=-1, top_p=1.0):
        self.max_rows, self.vocab = max_rows, vocab
        self.temperature, self.top_k, self.top_p = temperature, top_k, top_p
        self.states = torch.empty(max_rows * capi.SAMPLING_STATE_BYTES, dtype=torch.uint8, device=device)
        capi.sampling_setup_rand(seed, self.states)
        self.logits32 = torch.empty(max_rows, vocab, dtype=torch.float32, device=device)
        self.tokens = torch.empty(max_rows, dtype=torch.int32, device=device)
        self.scratch = (torch.empty(max_rows, vocab, dtype=torch.float32, device=device)
                        if vocab > capi.SAMPLING_REGISTER_VOCAB else None)

    def __call__(self, logits):
        """logits [S, V] -> tokens [S] int32 (a view valid until the next call)."""
        S, V = logits.shape
        assert S <= self.max_rows and V == self.vocab
        if logits.dtype == torch.float32 and logits.is_contiguous():
            x = logits
        else:
            x = self.logits32[:S]
            x.copy_(logits)
        out = self.tokens[:S]
        capi.sample(x, self.states[:S * capi.SAMPLING_STATE_BYTES], out, self.temperature, self.top_k, self.top_p,
                    scratch=None if self.scratch is None else self.scratch[:S])
        return out


__all__ = ["GpuSampler"]
