"""Python handle on the Qwen2-shaped decoder (include/kvc/qwen_model.h, kvc_qwen_* in the
C ABI): random-weight model on the device, greedy continuous-batching serving, one-prompt
prefill logits, and read-back of weight tensors (used by the CPU restatement in tests)."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._native import QwenConfigC, QwenStatsC, check, lib


@dataclass
class QwenConfig:
    layers: int = 24
    hidden: int = 896
    n_heads: int = 14
    n_kv_heads: int = 2
    head_dim: int = 64
    inter: int = 4864
    vocab: int = 151936
    eps: float = 1e-6
    theta: float = 1e6
    init_std: float = 0.02
    block_size: int = 16
    num_blocks: int = 10922
    max_batch: int = 32
    max_rows: int = 1024
    seed: int = 0
    step_path: int = 0  # 0: fused decode-step kernels for steps of <= 32 rows; 1: one kernel per op
    graph: int = 0  # 1: fused decode steps replay one captured HIP graph
    prefill_rows: int = 4096  # prompt rows stacked into one prefill forward
    chain: int = 0  # 1: linear layers between two attention launches as one launch (where allowed); 0: off

    def to_c(self) -> QwenConfigC:
        return QwenConfigC(self.layers, self.hidden, self.n_heads, self.n_kv_heads, self.head_dim, self.inter,
                           self.vocab, self.eps, self.theta, self.init_std, self.block_size, self.num_blocks,
                           self.max_batch, self.max_rows, self.seed, self.step_path, self.graph,
                           self.prefill_rows, self.chain)


class QwenModel:
    def __init__(self, cfg: QwenConfig):
        self.cfg = cfg
        self._c = cfg.to_c()
        h = C.c_void_p()
        check(lib().kvc_qwen_create(C.byref(self._c), C.byref(h)))
        self._h = h

    def close(self) -> None:
        if self._h:
            lib().kvc_qwen_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 -- interpreter shutdown
            pass

    def tensor(self, name: str, layer: int = 0) -> np.ndarray:
        """A weight copied to the host as fp16 (flat)."""
        p, n = C.c_void_p(), C.c_size_t()
        check(lib().kvc_qwen_tensor(self._h, name.encode(), layer, C.byref(p), C.byref(n)))
        out = np.empty(n.value // 2, np.float16)
        check(lib().kvc_memcpy_d2h(out.ctypes.data, p, n.value, None))
        check(lib().kvc_device_synchronize())
        return out

    def load_weights(self, directory) -> None:
        """Weights from the reference's dump format: manifest.tsv + weights.bin."""
        check(lib().kvc_qwen_load_weights(self._h, str(directory).encode()))

    def save_weights(self, directory) -> None:
        check(lib().kvc_qwen_save_weights(self._h, str(directory).encode()))

    def prefill_logits(self, tokens) -> tuple[int, np.ndarray]:
        t = np.ascontiguousarray(np.asarray(tokens, np.int32))
        logits = np.empty(self.cfg.vocab, np.float32)
        tok = C.c_int(0)
        check(lib().kvc_qwen_prefill_logits(self._h, t.ctypes.data, len(t), logits.ctypes.data, C.byref(tok)))
        return tok.value, logits

    def serve(self, prompts, gen_lens):
        """Greedy continuous batching; returns (list of generated token arrays, stats dict)."""
        off = np.concatenate([[0], np.cumsum([len(p) for p in prompts])]).astype(np.int32)
        flat = np.ascontiguousarray(np.concatenate([np.asarray(p, np.int32) for p in prompts]) if len(prompts)
                                    else np.zeros(0, np.int32))
        g = np.ascontiguousarray(np.asarray(gen_lens, np.int32))
        out = np.zeros(int(g.sum()), np.int32)
        st = QwenStatsC()
        check(lib().kvc_qwen_serve(self._h, len(prompts), off.ctypes.data, flat.ctypes.data, g.ctypes.data,
                                   out.ctypes.data, C.byref(st)))
        res, o = [], 0
        for n in g:
            res.append(out[o:o + n].copy())
            o += n
        return res, {"steps": st.steps, "finished": st.finished, "tokens": st.tokens,
                     "prompt_tokens": st.prompt_tokens, "wall_us": st.wall_us, "prefill_us": st.prefill_us,
                     "decode_us": st.decode_us, "graph_steps": st.graph_steps,
                     "graph_captures": st.graph_captures, "chain_launches": st.chain_launches}
