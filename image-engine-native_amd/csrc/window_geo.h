// window_geo.h -- window geometry shared by the window kernels (internal):
// the rolled window partition of crates/scunet-native/src/swin.rs and
// crates/birefnet-native/src/swin.rs over a map padded to whole windows.
#pragma once

#include <cstdint>

#include "ien_internal.h"

namespace ien {

// A block's window geometry (ien_windows plus what follows from it).
struct WinGeo {
  int window, shift, height, width;
  int ph, pw;  // the map padded to whole windows
  int wx;      // windows per row of windows
  int n;       // tokens per window
  long windows;
};

// Source token of window token i of window w, or -1 past the map's edge:
// ((wy W + i / W + shift) mod ph, (wx W + i % W + shift) mod pw).
__device__ __forceinline__ long win_source(const WinGeo &g, long w, int i) {
  const int wy = (int)(w / g.wx), wxi = (int)(w - (long)wy * g.wx);
  int y = wy * g.window + i / g.window + g.shift;
  int x = wxi * g.window + i % g.window + g.shift;
  if (y >= g.ph) y -= g.ph;  // shift < window <= ph: one wrap at most
  if (x >= g.pw) x -= g.pw;
  if (y >= g.height || x >= g.width) return -1;
  return (long)y * g.width + x;
}

// The same in 32-bit arithmetic (window counts and maps under 2^31).
__device__ __forceinline__ int win_source(const WinGeo &g, int w, int i) {
  const int wy = w / g.wx, wxi = w - wy * g.wx;
  int y = wy * g.window + i / g.window + g.shift;
  int x = wxi * g.window + i % g.window + g.shift;
  if (y >= g.ph) y -= g.ph;
  if (x >= g.pw) x -= g.pw;
  if (y >= g.height || x >= g.width) return -1;
  return y * g.width + x;
}

// swin.rs:171-176: 1 for a window last in its row, 2 last in its column.
__device__ __forceinline__ int win_class(const WinGeo &g, long w) {
  if (g.shift == 0) return 0;
  const long rows = g.windows / g.wx;
  return (int)(w % g.wx == g.wx - 1) + 2 * (int)(w / g.wx == rows - 1);
}

inline ien_status geometry(const ien_windows *w, WinGeo *g) {
  IEN_CHECK(w, IEN_ERR_INPUT, "null windows");
  IEN_CHECK(w->window >= 1 && w->window * w->window <= 256, IEN_ERR_INPUT,
            "window %d (at most 16 x 16 tokens)", w->window);
  IEN_CHECK(w->shift >= 0 && w->shift < w->window, IEN_ERR_INPUT, "shift %d of window %d",
            w->shift, w->window);
  IEN_CHECK(w->height >= 1 && w->width >= 1, IEN_ERR_INPUT, "map %d x %d", w->height, w->width);
  g->window = w->window;
  g->shift = w->shift;
  g->height = w->height;
  g->width = w->width;
  g->ph = (w->height + w->window - 1) / w->window * w->window;
  g->pw = (w->width + w->window - 1) / w->window * w->window;
  g->wx = g->pw / w->window;
  g->n = w->window * w->window;
  g->windows = (long)(g->ph / w->window) * g->wx;
  return IEN_OK;
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace ien
