"""Request lifecycle restated from kunserve/request.py:368-462 (test code
only): chunked prefill advances prefill_[begin|end]_index; after the prompt
each step decodes one token. Gives each step's pforward row arguments and
the pages the block manager holds for the row."""
from __future__ import annotations


class Request:
    def __init__(self, prompt_len: int, chunk: int):
        self.prompt_len, self.chunk = prompt_len, chunk
        self.begin = self.end = 0
        self.outputs = 0

    def context_stage(self) -> bool:
        return self.outputs == 0

    def step_args(self, use_tensor_cores: bool, page_size: int):
        """(first_token_index, q_len, flag, real stage, pages in the table).

        get_first_new_token_index (request.py:447-462); the flag of
        get_is_context_stage (request.py:667-670); a context row's table is
        cut to ceil(prefill_end_index / bs) pages (block_manager.py:786-795),
        a decode row holds ceil(get_num_tokens() / bs) pages
        (block_manager.py:493-500, request.py:414-423)."""
        ctx = self.context_stage()
        if ctx:
            self.begin = self.end
            self.end = min(self.begin + self.chunk, self.prompt_len)
            first, ql, tokens = self.begin, self.end - self.begin, self.end
        else:
            first, ql = self.prompt_len + self.outputs, 1
            tokens = self.prompt_len + self.outputs
        flag = 1 if (use_tensor_cores or ctx) else 0
        return first, ql, flag, int(ctx), -(-tokens // page_size)

    def finish_step(self) -> None:
        if self.context_stage() and self.end < self.prompt_len:
            return
        self.outputs += 1
