// Workspace policy of the plugin products (jm_q4_gemm_f32, jm_q4_gemv_f32),
// host code only (the CPU tests compile it on its own).  Each (device,
// stream) keeps one persistent buffer, and a call either reuses it, grows
// it, or (under stream capture) takes a stream-ordered allocation that it
// frees after its kernels:
//   - a graph being captured must not bake in the persistent buffer: a later
//     eager call on the stream that needs more space would replace it while
//     the graph still points at it;
//   - a grown buffer's predecessor is retired, not freed: another host thread
//     may have taken its pointer for kernels it has not enqueued yet, and a
//     captured graph may still use it.  Retired buffers live until the
//     process ends; with the growth below they total at most the final size.
#pragma once

#include <stddef.h>

namespace jm {

enum class WsAction { Reuse, StreamOrdered, Grow };

inline WsAction plugin_ws_action(size_t have_bytes, size_t need, bool capturing) {
    if (capturing) return WsAction::StreamOrdered;
    if (have_bytes >= need) return WsAction::Reuse;
    return WsAction::Grow;
}

// bytes to allocate when growing: at least 1 MiB and at least twice the
// buffer it replaces, so that a stream's retired buffers sum to less than
// its current one
inline size_t plugin_ws_grow(size_t have_bytes, size_t need) {
    size_t g = need > ((size_t)1 << 20) ? need : ((size_t)1 << 20);
    if (g < 2 * have_bytes) g = 2 * have_bytes;
    return g;
}

}  // namespace jm
