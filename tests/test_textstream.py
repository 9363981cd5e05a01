"""CPU: the completion text helpers (mlx_dspark/textstream.py) against the reference's own test
vectors for its streaming, stop-string, finish-reason and chat-template helpers
(tests/test_generate_helpers.py:17-142, :173-181), held here as data: the stop strings and the
text each round adds, with the streamed text, the final text and whether the stream closed.
The tokenizer renders ids as the characters with those code points, as the reference's tests'
stand-in does."""

import pytest

from mlx_dspark.textstream import StopStreaming, TextStream, _id_list, encode_prompt, eos_token_ids


class CodepointTok:
    def decode(self, ids):
        return "".join(chr(i) for i in ids)


def _run(stop, rounds, eos=frozenset(), on_text=None):
    chunks = []
    st = TextStream(CodepointTok(), set(eos), on_text or chunks.append, stop)
    out = []
    for r in rounds:
        out += [ord(c) for c in r]
        st.feed(out)
        if st.closed:
            break
    st.close()
    return "".join(chunks), st.text, st.closed


# (stop strings, text added per round) -> (streamed text, final text, closed)
VECTORS = [
    (None, ["Hel", "lo ", "world"], ("Hello world", "Hello world", False)),        # :31-33
    (["STOP"], ["abc", "deSTOPxyz"], ("abcde", "abcde", True)),                     # :36-39
    (["STOP"], ["abST", "OPcd"], ("ab", "ab", True)),                               # :42-45
    (["END", "STOP"], ["xxSTOPyyENDzz"], ("xx", "xx", True)),                       # :48-50
]


@pytest.mark.parametrize("stop,rounds,want", VECTORS)
def test_reference_stream_vectors(stop, rounds, want):
    assert _run(stop, rounds) == want


def test_incremental_feed_matches_full_decode():
    # tests/test_generate_helpers.py:53-67: one id per feed, a trailing eos id never renders
    msg = "incremental detokenization, olé! → 対応"
    chunks = []
    st = TextStream(CodepointTok(), {9999}, chunks.append, None)
    out = []
    for c in msg:
        out.append(ord(c))
        st.feed(out)
    out.append(9999)
    st.feed(out)
    st.close()
    assert "".join(chunks) == msg and st.text == msg and st.result_text(out) == msg


def test_stop_streaming_from_on_text_closes_the_stream():
    # tests/test_generate_helpers.py:108-128
    chunks = []

    def on_text(piece):
        chunks.append(piece)
        if sum(map(len, chunks)) >= 3:
            raise StopStreaming()

    streamed, text, closed = _run(None, list("abcdefgh"), on_text=on_text)
    assert closed and "".join(chunks) == "abc" and text.startswith("abc")


def test_nothing_of_a_stop_string_is_streamed_at_any_split():
    # every split of the text into two rounds, and one character per round: the streamed text is
    # the text before the earliest stop string, never more
    text, stops = "one two <|end|> three", ["<|end|>", "two!"]
    want = "one two "
    for cut in range(len(text) + 1):
        assert _run(stops, [text[:cut], text[cut:]])[:2] == (want, want), cut
    assert _run(stops, list(text))[:2] == (want, want)


def test_held_back_tail_is_released_when_no_stop_follows():
    # "ST" could begin "STOP": it waits until the next round shows it does not, then streams
    chunks = []
    st = TextStream(CodepointTok(), set(), chunks.append, ["STOP"])
    out = [ord(c) for c in "abST"]
    st.feed(out)
    assert "".join(chunks) == "ab"
    out += [ord(c) for c in "ARx"]
    st.feed(out)
    assert "".join(chunks) == "abSTARx" and not st.closed


def test_finish_reason():
    # tests/test_generate_helpers.py:135-142: eos last -> stop; a stop string -> stop; the cap
    # reached -> length; under the cap without eos -> stop
    open_ = TextStream(CodepointTok(), {9}, None, None)
    assert open_.finish_reason([1, 2, 3], 3, 9) == "stop"
    assert open_.finish_reason([1, 2, 3], 3, 5) == "length"
    assert open_.finish_reason([1, 2], 3, 5) == "stop"
    hit = TextStream(CodepointTok(), {9}, None, ["b"])
    hit.feed([ord("a"), ord("b")])
    assert hit.closed and hit.finish_reason([1, 2, 3], 100, 5) == "stop"


def test_template_result_shapes():
    # tests/test_generate_helpers.py:173-181, and an encoding object with .ids
    class BatchEncoding(dict):
        pass

    class Encoding:
        ids = [3, 1]

    assert _id_list([1, 2, 3]) == [1, 2, 3]
    assert _id_list([[4, 5, 6]]) == [4, 5, 6]
    assert _id_list(BatchEncoding(input_ids=[[7, 8, 9]])) == [7, 8, 9]
    assert _id_list(Encoding()) == [3, 1]


def test_prompt_encoding_and_end_ids():
    class Tok:
        chat_template = "t"
        eos_token_id = 2
        unk_token_id = 0

        def encode(self, s):
            return [ord(c) for c in s]

        def apply_chat_template(self, messages, add_generation_prompt=True, tools=None):
            return [[1] + self.encode(messages[0]["content"]) + ([4] if add_generation_prompt else [])]

        def convert_tokens_to_ids(self, t):
            return {"<|im_end|>": 7, "<eos>": 0}.get(t, -1)

    t = Tok()
    assert encode_prompt(t, "hi") == [1, 104, 105, 4]
    assert encode_prompt(t, "hi", use_chat=False) == [104, 105]
    assert eos_token_ids(t) == {2, 7}          # <eos> resolves to the unknown id: not an end id
