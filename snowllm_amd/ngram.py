# SPDX-License-Identifier: Apache-2.0
# The function name, arguments and result here follow snowllm/ngram.py (SPDX-FileCopyrightText:
# Copyright contributors to the SnowLLM project), which this module keeps so that the
# reference's sampler masks the same tokens with it.
"""No-repeat-n-gram bans (snowllm/ngram.py; used by snowllm/engine/sampler.py:146-168)."""


def banned_ngram_tokens(tokens, size):
    """The tokens that would complete an n-gram of `size` already present in `tokens`: every
    token that followed an earlier occurrence of the last size - 1 tokens, ascending. size 1
    bans every token seen; size <= 0, or fewer than size - 1 tokens, bans nothing."""
    if size <= 0 or len(tokens) + 1 < size:
        return []
    n = size - 1
    tail = tuple(tokens[len(tokens) - n:]) if n else ()
    out = set()
    for end in range(n, len(tokens)):
        if tuple(tokens[end - n:end]) == tail:
            out.add(tokens[end])
    return sorted(out)
