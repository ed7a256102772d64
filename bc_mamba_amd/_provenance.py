"""What the extraction already knows about the tensors it returns, kept on
them so that later calls of the drop-in API need not recompute it.

* The event index (bitmask [rows, words] + tile table [rows, tiles+1]) is
  built by the extraction's fill anyway. The restore forward / backward and
  the gather backward of the same events read it instead of rebuilding it
  from (time_steps, cu_seqlens) or zero-filling and scattering.
* The channel-length maximum is read on the host by the extraction. A scan
  whose max_seqlen covers it needs no device-side length report (and no host
  sync to read one).

Both are Python attributes of the returned tensors, valid only while those
tensors are unchanged: a record keeps the data pointer, size and version
counter of every tensor it depends on, and a weak reference to each one
other than its holder. A dependency that has been freed voids the record,
so a match cannot come from another tensor that reuses the memory (the
holder's own memory lives as long as the record), and a record keeps no
tensor alive. A call whose tensors do not match computes what it needs, as
for any other input.
"""
import weakref

_INDEX = "_bcm_event_index"
_MAXLEN = "_bcm_max_seqlen"


def _sig(t):
    return (t.data_ptr(), t.numel(), t._version)


class EventIndex:
    """(bitmask, tile_start) of one extraction's events, kept on its
    time_steps and tied to its channel_ids and cu_seqlens and to seqlen."""

    __slots__ = ("bitmask", "tile_start", "seqlen", "ch", "cu", "sigs", "bm_ver")

    def __init__(self, bitmask, tile_start, seqlen, time_steps, channel_ids, cu_seqlens):
        self.bitmask, self.tile_start, self.seqlen = bitmask, tile_start, int(seqlen)
        self.ch, self.cu = weakref.ref(channel_ids), weakref.ref(cu_seqlens)
        self.sigs = (_sig(time_steps), _sig(channel_ids), _sig(cu_seqlens))
        self.bm_ver = (bitmask._version, tile_start._version)

    @staticmethod
    def _same(ref, given, sig):
        """given describes the data the record was made for: the recorded
        tensor is still alive and unchanged, and given shares its data."""
        rec = ref()
        return rec is not None and _sig(rec) == sig and _sig(given) == sig

    def matches(self, time_steps, cu_seqlens, seqlen, channel_ids=None):
        if int(seqlen) != self.seqlen or (self.bitmask._version, self.tile_start._version) != self.bm_ver:
            return False
        if _sig(time_steps) != self.sigs[0]:
            return False
        if cu_seqlens is not None and not self._same(self.cu, cu_seqlens, self.sigs[2]):
            return False
        if channel_ids is not None and not self._same(self.ch, channel_ids, self.sigs[1]):
            return False
        return True


def attach_event_index(time_steps, channel_ids, cu_seqlens, seqlen, bitmask, tile_start):
    """Record on time_steps the index the extraction built for its events."""
    setattr(time_steps, _INDEX, EventIndex(bitmask, tile_start, seqlen, time_steps, channel_ids, cu_seqlens))


def event_index_for(time_steps, cu_seqlens, seqlen, channel_ids=None):
    """(bitmask, tile_start) recorded on time_steps when it still describes
    these tensors (and channel_ids, when given), else None."""
    idx = getattr(time_steps, _INDEX, None)
    if idx is None or not idx.matches(time_steps, cu_seqlens, seqlen, channel_ids):
        return None
    return idx.bitmask, idx.tile_start


def attach_max_seqlen(cu_seqlens, max_seqlen):
    """Record on cu_seqlens the longest channel of its offsets."""
    setattr(cu_seqlens, _MAXLEN, (int(max_seqlen), _sig(cu_seqlens)))


def max_seqlen_of(cu_seqlens):
    """The longest channel recorded on cu_seqlens while it is unchanged, else
    None."""
    rec = getattr(cu_seqlens, _MAXLEN, None)
    if rec is None or _sig(cu_seqlens) != rec[1]:
        return None
    return rec[0]


def covers_max_seqlen(cu_seqlens, max_seqlen):
    """True when cu_seqlens carries its longest channel and max_seqlen is at
    least that long (no channel can overrun it)."""
    m = max_seqlen_of(cu_seqlens)
    return m is not None and int(max_seqlen) >= m
