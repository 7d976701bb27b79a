// Attention masks and positions that the reference's model graphs build on the
// host before handing them to ggml's attention ops, in the forms the paged
// attention takes (u8 "visible" masks for EMB_MASK_TOKEN, f32 additive masks for
// EMB_MASK_ADD) and in the reference's own forms (f16 / f32 additive, 0 or
// -inf) for the ggml-descriptor face.
//
//   HY-VLA   make_visual_patch_groups / make_prefix_mask
//            (models/hy_vla.cpp:1251-1306) and the expert-with-prefix mask
//            (:2831-2843);
//   GR00T    the DiT cross-attention text / image masks (models/groot_n1.cpp
//            :708-716) and which DiT layer uses which (:656-661);
//   SmolVLA  the prefix, expert self-attention and cross-attention masks
//            (models/smolvla.cpp:696-725) and the RoPE positions (:680-688).
#include <cstring>
#include <vector>

#include "emb_common.h"

namespace {

constexpr uint16_t F16_ZERO = 0x0000u;
constexpr uint16_t F16_NEG_INF = 0xFC00u;

inline void put(uint8_t *allow, uint16_t *mask_f16, int64_t i, bool vis) {
    if (allow) allow[i] = vis ? 1 : 0;
    if (mask_f16) mask_f16[i] = vis ? F16_ZERO : F16_NEG_INF;
}

}  // namespace

extern "C" {

// Visual patch groups: maximal runs of tokens with a nonzero modality flag,
// where a single zero between two runs does not end the group (the zero token
// itself joins none) and two or more zeros do.  group_of[i] = group index, or
// -1 for a token in no group.  Returns the number of groups.
int32_t emb_hy_patch_groups(const int32_t *modality_mask, int32_t n, int32_t *group_of) {
    EMB_CHECK_ARG(modality_mask && group_of && n >= 0, "bad argument");
    int32_t groups = 0;
    bool open = false;  // a group has members and is still open
    int32_t i = 0;
    for (int32_t k = 0; k < n; ++k) group_of[k] = -1;
    while (i < n) {
        if (modality_mask[i] == 0) {
            const int32_t z0 = i;
            while (i < n && modality_mask[i] == 0) ++i;
            if (i - z0 >= 2 && open) {
                ++groups;
                open = false;
            }
            continue;
        }
        while (i < n && modality_mask[i] != 0) group_of[i++] = groups;
        open = true;
    }
    return open ? groups + 1 : groups;
}

// Prefix mask [n][n], row = query, column = key: causal (key <= query), except
// that among tokens in patch groups a key is visible exactly when it is in the
// query's own group (either order).  group_of NULL: causal only (the text-only
// generation call, :2131).  allow (1 = visible) and/or mask_f16 (the
// reference's additive F16 values 0 / -inf) may each be NULL.
int emb_hy_prefix_mask(int64_t n, const int32_t *group_of, uint8_t *allow, uint16_t *mask_f16) {
    EMB_CHECK_ARG(n > 0 && (allow || mask_f16), "bad argument");
    for (int64_t r = 0; r < n; ++r) {
        const int32_t gr = group_of ? group_of[r] : -1;
        for (int64_t c = 0; c < n; ++c) {
            const int32_t gc = group_of ? group_of[c] : -1;
            const bool vis = gr >= 0 && gc >= 0 ? gr == gc : c <= r;
            put(allow, mask_f16, r * n + c, vis);
        }
    }
    return EMB_OK;
}

// Expert-with-prefix mask [n_suf][n_pref + n_suf]: every prefix key visible;
// among the suffix keys row 0 (the state token) sees only itself, the other
// rows see the whole suffix.
int emb_hy_suffix_mask(int64_t n_pref, int64_t n_suf, uint8_t *allow, uint16_t *mask_f16) {
    EMB_CHECK_ARG(n_pref >= 0 && n_suf > 0 && (allow || mask_f16), "bad argument");
    const int64_t n_total = n_pref + n_suf;
    for (int64_t r = 0; r < n_suf; ++r)
        for (int64_t c = 0; c < n_total; ++c) {
            const bool vis = c < n_pref || r != 0 || c == n_pref;
            put(allow, mask_f16, r * n_total + c, vis);
        }
    return EMB_OK;
}

// Which mask DiT layer `layer` cross-attends with: odd layers are
// self-attention (0, no mask); even layers alternate between the text mask (1)
// and the image mask (2) with period 2 * attend_text_every_n_blocks, the text
// mask first.
int emb_groot_layer_mask_kind(int32_t layer, int32_t attend_text_every_n_blocks) {
    EMB_CHECK_ARG(layer >= 0 && attend_text_every_n_blocks > 0, "bad argument");
    if (layer % 2 == 1) return 0;
    return layer % (2 * attend_text_every_n_blocks) == 0 ? 1 : 2;
}

// Cross-attention masks [n_q][n_keys], f32 additive (0 / -inf): text_mask
// shows the valid non-image backbone keys, image_mask the valid image keys;
// every query row is the same.  Either output may be NULL.
int emb_groot_cross_masks(const int32_t *attention_mask, const int32_t *image_flags, int64_t n_keys, int64_t n_q,
                          float *text_mask, float *image_mask) {
    EMB_CHECK_ARG(attention_mask && image_flags && n_keys > 0 && n_q > 0 && (text_mask || image_mask),
                  "bad argument");
    const float neg_inf = -__builtin_inff();
    for (int64_t q = 0; q < n_q; ++q)
        for (int64_t k = 0; k < n_keys; ++k) {
            const bool valid = attention_mask[k] != 0, img = image_flags[k] != 0;
            if (text_mask) text_mask[q * n_keys + k] = valid && !img ? 0.0f : neg_inf;
            if (image_mask) image_mask[q * n_keys + k] = valid && img ? 0.0f : neg_inf;
        }
    return EMB_OK;
}

// SmolVLA masks, f32 additive (0 / -inf); any output may be NULL.
//   prefix_mask [n_prefix][n_prefix]: invalid (padding) keys hidden, and the
//     last prefix token (the state) hidden from every other query;
//   full_mask [n_suf][n_prefix + n_suf]: invalid prefix keys hidden, causal
//     within the action suffix;
//   cross_mask [n_suf][n_prefix]: invalid prefix keys hidden.
int emb_smolvla_masks(const uint8_t *prefix_valid, int64_t n_prefix, int64_t n_suf, float *prefix_mask,
                      float *full_mask, float *cross_mask) {
    EMB_CHECK_ARG(prefix_valid && n_prefix > 0 && n_suf > 0, "bad argument");
    const float neg_inf = -__builtin_inff();
    if (prefix_mask)
        for (int64_t q = 0; q < n_prefix; ++q)
            for (int64_t k = 0; k < n_prefix; ++k)
                prefix_mask[q * n_prefix + k] =
                    !prefix_valid[k] || (q < n_prefix - 1 && k == n_prefix - 1) ? neg_inf : 0.0f;
    const int64_t n_total = n_prefix + n_suf;
    for (int64_t q = 0; q < n_suf; ++q) {
        for (int64_t k = 0; k < n_prefix; ++k) {
            const float v = prefix_valid[k] ? 0.0f : neg_inf;
            if (full_mask) full_mask[q * n_total + k] = v;
            if (cross_mask) cross_mask[q * n_prefix + k] = v;
        }
        if (full_mask)
            for (int64_t k = 0; k < n_suf; ++k) full_mask[q * n_total + n_prefix + k] = k > q ? neg_inf : 0.0f;
    }
    return EMB_OK;
}

// SmolVLA RoPE positions: prefix token i sits at (valid tokens up to and
// including i) - 1, at least 0; suffix token i at (valid prefix tokens) + i;
// the cross-attention queries at i.  Any output may be NULL.
int emb_smolvla_positions(const uint8_t *prefix_valid, int64_t n_prefix, int64_t n_suf, int32_t *prefix_pos,
                          int32_t *suffix_pos, int32_t *cross_pos) {
    EMB_CHECK_ARG(prefix_valid && n_prefix > 0 && n_suf >= 0, "bad argument");
    int32_t pos = -1;
    for (int64_t i = 0; i < n_prefix; ++i) {
        if (prefix_valid[i]) ++pos;
        if (prefix_pos) prefix_pos[i] = pos > 0 ? pos : 0;
    }
    for (int64_t i = 0; i < n_suf; ++i) {
        if (suffix_pos) suffix_pos[i] = pos + 1 + (int32_t)i;
        if (cross_pos) cross_pos[i] = (int32_t)i;
    }
    return EMB_OK;
}

}  // extern "C"
