"""tokenizer.Tokenizer (tokenizer/tokenizer.go) on the native tokenizer of
libindecis_hip.so (host code; no GPU is touched): Encode, EncodeMax,
EncodePair, EncodeOffsets, and encode_batch, which tokenizes many texts on
several threads into the packed ids/offsets the encoder takes."""
import ctypes as C

import numpy as np

from . import _lib


def _b(text):
    return text.encode("utf-8") if isinstance(text, str) else bytes(text)


class Tokenizer:
    def __init__(self, path):
        h = C.c_void_p()
        _lib.check(_lib.lib().ixh_tokenizer_load(str(path).encode(), C.byref(h)))
        self._h = h
        v, b, e, p = (C.c_int32() for _ in range(4))
        _lib.check(_lib.lib().ixh_tokenizer_info(h, C.byref(v), C.byref(b), C.byref(e), C.byref(p)))
        self.vocab_size, self.bos_id, self.eos_id, self.pad_id = v.value, b.value, e.value, p.value

    def close(self):
        if self._h:
            _lib.lib().ixh_tokenizer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _ids(self, call):
        n = C.c_int64(0)
        _lib.check(call(None, 0, C.byref(n)))
        out = np.zeros(n.value, np.int32)
        _lib.check(call(out.ctypes.data_as(C.c_void_p), n.value, C.byref(n)))
        return out

    def encode(self, text, max_len=None):
        """Encode (max_len None) or EncodeMax (tokenizer.go:479-495)."""
        t = _b(text)
        max_len = -1 if max_len is None else max_len
        return self._ids(lambda o, cap, n: _lib.lib().ixh_tokenizer_encode(self._h, t, len(t), max_len, o, cap, n))

    def encode_pair(self, context, text, max_len=0):
        """EncodePair (tokenizer.go:497-518)."""
        c, t = _b(context), _b(text)
        return self._ids(lambda o, cap, n: _lib.lib().ixh_tokenizer_encode_pair(
            self._h, c, len(c), t, len(t), max_len, o, cap, n))

    def encode_offsets(self, text):
        """EncodeOffsets (tokenizer.go:525-540): (ids, [(start, end)])."""
        t = _b(text)
        L = _lib.lib()
        n = C.c_int64(0)
        _lib.check(L.ixh_tokenizer_encode_offsets(self._h, t, len(t), None, None, None, 0, C.byref(n)))
        ids = np.zeros(n.value, np.int32)
        st, en = np.zeros(n.value, np.int64), np.zeros(n.value, np.int64)
        p = lambda a: a.ctypes.data_as(C.c_void_p)
        _lib.check(L.ixh_tokenizer_encode_offsets(self._h, t, len(t), p(ids), p(st), p(en), n.value, C.byref(n)))
        return ids, list(zip(st.tolist(), en.tolist()))

    def encode_batch(self, texts, max_len=None, threads=0):
        """EncodeMax (Encode with max_len None) of every text, on `threads`
        threads (0: one per core): (ids laid end to end, offs [n+1]) as
        ixh_encode_seqs takes them."""
        max_len = -1 if max_len is None else max_len
        bs = [_b(t) for t in texts]
        n = len(bs)
        arr = (C.c_char_p * max(n, 1))(*bs)
        lens = np.array([len(b) for b in bs] or [0], np.int64)
        offs = np.zeros(n + 1, np.int32)
        L = _lib.lib()
        p = lambda a: a.ctypes.data_as(C.c_void_p)
        # One pass into room for the most a text can give: 3 ids per byte
        # (a byte fallback of ' ' -> U+2581), 3 for a leading U+2581, and the
        # template's specials; a second pass only if the template holds more
        # than 16 of them.
        bound = 3 * lens[:n] + 3 + 16
        if max_len >= 0:
            bound = np.minimum(bound, max(max_len, 16))
        ids = np.empty(int(bound.sum()), np.int32)
        rc = L.ixh_tokenizer_encode_batch(self._h, C.cast(arr, C.c_void_p), p(lens), n, max_len, threads,
                                          p(ids), ids.size, p(offs))
        if rc == _lib.IXH_EINVAL and n and offs[-1] > ids.size:
            ids = np.empty(int(offs[-1]), np.int32)
            rc = L.ixh_tokenizer_encode_batch(self._h, C.cast(arr, C.c_void_p), p(lens), n, max_len, threads,
                                              p(ids), ids.size, p(offs))
        _lib.check(rc)
        return ids[:offs[-1]], offs
