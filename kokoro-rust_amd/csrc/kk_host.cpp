// kk_host.cpp -- host-only rules of the C ABI: durations_from_logits and the ragged layout tables
// (the bit-exact integer contract of the path), and the checks of an ids-level item.  Plain C++,
// built into the library and, for the sanitizer tests, on its own.
#include "kk_host.h"

#include <cmath>

namespace kk {

std::string ids_item_error(const kk_item& it, int b) {
    const std::string sb = std::to_string(b);
    if (it.ids == nullptr || it.ref_s == nullptr) return "item " + sb + ": null input";
    if (it.n_ids < 2 || it.n_ids > 512) return "item " + sb + ": input_ids length outside [2, 512]";
    if (!(std::isfinite(it.speed) && it.speed > 0.f)) return "item " + sb + ": speed must be positive and finite";
    for (int i = 0; i < it.n_ids; i++)  // the message is built only for a failing id
        if (it.ids[i] < 0 || it.ids[i] >= 178)
            return "item " + sb + ": token id " + std::to_string(it.ids[i]) + " out of range";
    if (it.noise_kind != KK_NOISE_COUNTER && it.noise_kind != KK_NOISE_FIXED) return "item " + sb + ": unknown noise kind";
    return "";
}

}  // namespace kk

using kk::kGapN;

extern "C" {

int kk_durations_from_logits(const float* logits, int t, float speed, int64_t* out) {
    if (!logits || !out || t < 0 || !(speed > 0.f) || !std::isfinite(speed)) return KK_ERR_INVALID;
    // src/model.rs:90-99 with src/ops.rs:49-51: f32 sigmoid, left-to-right f32 sum, ties to even
    for (int i = 0; i < t; i++) {
        float s = 0.f;
        for (int j = 0; j < 50; j++) {
            volatile float e = std::exp(-logits[i * 50 + j]);
            s = s + 1.0f / (1.0f + (float)e);
        }
        const float d = std::nearbyint(s / speed);
        // `d as i64` in Rust saturates: NaN -> 0, at or past 2^63 -> i64::MAX (the sum is >= 0)
        const int64_t di = std::isnan(d) ? 0 : d >= 9.223372036854775808e18f ? INT64_MAX : (int64_t)d;
        out[i] = di < 1 ? 1 : di;
    }
    return KK_OK;
}

int64_t kk_layout_frames(const int64_t* nfs, int n, int64_t* a_out) {
    if (!nfs || !a_out || n <= 0) return KK_ERR_INVALID;
    int64_t ln = 0;
    for (int b = 0; b < n; b++) {
        if (nfs[b] < 0 || nfs[b] > ((int64_t)1 << 40)) return KK_ERR_INVALID;
        a_out[b] = ln;
        ln += nfs[b] + kGapN;
    }
    return ln;
}

int kk_layout_col_item(int64_t l, const int64_t* start, const int64_t* len, int n, int32_t* col_item) {
    if (!start || !len || !col_item || l < 0) return KK_ERR_INVALID;
    for (int64_t t = 0; t < l; t++) col_item[t] = -1;
    for (int b = 0; b < n; b++) {
        if (start[b] < 0 || len[b] < 0 || start[b] > l || len[b] > l - start[b]) return KK_ERR_INVALID;
        for (int64_t t = start[b]; t < start[b] + len[b]; t++) {
            if (col_item[t] >= 0) return KK_ERR_INVALID;
            col_item[t] = b;
        }
    }
    return KK_OK;
}

int kk_layout_src_row(const int64_t* const* dur, const int32_t* n_tok, int n, const int64_t* tstart, const int64_t* a,
                      int64_t ln, int32_t* src_row) {
    if (!dur || !n_tok || !tstart || !a || !src_row || ln < 0) return KK_ERR_INVALID;
    for (int64_t t = 0; t < ln; t++) src_row[t] = -1;
    for (int b = 0; b < n; b++) {
        if (a[b] < 0 || n_tok[b] < 0 || (n_tok[b] > 0 && !dur[b])) return KK_ERR_INVALID;
        int64_t f = a[b];
        for (int tok = 0; tok < n_tok[b]; tok++)
            for (int64_t r = 0; r < dur[b][tok]; r++) {
                if (f >= ln) return KK_ERR_INVALID;
                src_row[f++] = (int32_t)(tstart[b] + tok);
            }
    }
    return KK_OK;
}

}  // extern "C"
