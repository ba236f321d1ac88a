// Host-side producers of the attention path's inputs: the M-RoPE positions of a record and the
// packing of queued records into one micro-batch (cu_seqlens). Plain C++, no device code.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "clef_hip_attn.h"

namespace {
bool rfail(char *err, size_t errlen, const char *fmt, ...) {
    if (err && errlen) {
        const int n = snprintf(err, errlen, "hip: ");
        if (n > 0 && (size_t)n < errlen) {
            va_list ap;
            va_start(ap, fmt);
            vsnprintf(err + n, errlen - (size_t)n, fmt, ap);
            va_end(ap);
        }
    }
    return false;
}
}  // namespace

extern "C" {

// clef_record.c:938-962 (clef_record_positions): a record that carries its own positions
// (pos3_given, the reference's r->pos3, 939-942) has them copied; otherwise text tokens take
// (p, p, p) with p counting up from 0, and a vision span covers the merged grid
// (grid_h / merge) x (grid_w / merge) row-major, token (y, x) taking (p, p + y, p + x), after
// which p advances by the larger merged side.
bool clef_hip_record_positions(int T, const int32_t *pos3_given, const int32_t *span_start,
                               const int32_t *span_grid_h, const int32_t *span_grid_w, int n_spans, int merge,
                               int32_t *pos3, char *err, size_t errlen) {
    if (T < 0 || (T && !pos3)) return rfail(err, errlen, "bad record position arguments");
    if (pos3_given) {
        if (T) memmove(pos3, pos3_given, (size_t)T * 3 * sizeof(int32_t));
        return true;
    }
    if (n_spans < 0 || merge <= 0 || (n_spans && (!span_start || !span_grid_h || !span_grid_w)))
        return rfail(err, errlen, "bad record position arguments");
    int32_t cur = 0;
    int t = 0, next = 0;
    while (t < T) {
        if (next < n_spans && span_start[next] == t) {
            const int gh = span_grid_h[next], gw = span_grid_w[next];
            if (gh <= 0 || gw <= 0 || gh % merge || gw % merge)
                return rfail(err, errlen, "span %d grid %dx%d is not a positive multiple of the merge %d", next, gh, gw, merge);
            const int h = gh / merge, w = gw / merge;
            if ((long)t + (long)h * w > T) return rfail(err, errlen, "span %d runs past the record's %d tokens", next, T);
            for (int y = 0; y < h; y++)
                for (int x = 0; x < w; x++, t++) {
                    pos3[3 * t] = cur;
                    pos3[3 * t + 1] = cur + y;
                    pos3[3 * t + 2] = cur + x;
                }
            cur += h > w ? h : w;
            next++;
        } else {
            if (next < n_spans && span_start[next] < t)
                return rfail(err, errlen, "span %d starts at token %d, inside or before what precedes it", next, span_start[next]);
            pos3[3 * t] = pos3[3 * t + 1] = pos3[3 * t + 2] = cur;
            cur++;
            t++;
        }
    }
    if (next < n_spans) return rfail(err, errlen, "span %d starts at token %d, past the record's %d tokens", next, span_start[next], T);
    return true;
}

// clef_server.c:311-327: first in, first out; the head of the queue is always taken, then the
// next requests while fewer than max_batch are taken and their tokens stay within max_tokens.
// A request with a prefix-cache key (keyed[i] != 0) runs alone and stops the batch behind it.
int clef_hip_pack_batch(const int32_t *lengths, const uint8_t *keyed, int n_queue, int max_batch,
                        long max_tokens, int32_t *cu_seqlens) {
    if (!lengths || !cu_seqlens || n_queue <= 0 || max_batch <= 0) return 0;
    const bool head_keyed = keyed && keyed[0];
    int n = 0;
    long toks = 0;
    cu_seqlens[0] = 0;
    while (n < n_queue && n < max_batch &&
           (n == 0 || (!head_keyed && !(keyed && keyed[n]) && toks + lengths[n] <= max_tokens))) {
        toks += lengths[n];
        cu_seqlens[n + 1] = (int32_t)toks;
        n++;
    }
    return n;
}

}  // extern "C"
