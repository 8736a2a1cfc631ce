// kanso_oracle.cpp — CPU restatement of kanso-infer's attention-path arithmetic.
//
// TEST INFRASTRUCTURE ONLY: the checker the parity tests, smoke() and bench.py's
// cpu_baseline leg use. Nothing in the product links or loads it.
//
// Build: oracle/Makefile (g++ -O3 -march=native -ffp-contract=off -fopenmp). The
// no-contraction flag matters: Rust evaluates `a * b + c` as two rounded operations,
// and the quantizers below must round exactly like the Rust source to be bit-exact.

#include "kanso_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

// Rust f32::round: half away from zero. C roundf has the same definition.
inline float rust_round(float x) { return std::round(x); }

// `as i8` after an explicit clamp to the i8 range is a truncating conversion of an
// integral float, i.e. exact.
inline int8_t clamp_i8(float x, float lo, float hi) {
    return static_cast<int8_t>(std::min(std::max(x, lo), hi));
}

struct DequantView {
    uint32_t kv_dtype, bs, hkv, d;
    const void* pool;
    const void* scales;
    // Writes the f32 row of (block, offset, head) into out[d].
    void row(uint32_t block, uint32_t off, uint32_t head, float* out) const {
        const size_t row_idx = (static_cast<size_t>(block) * bs + off) * hkv + head;
        if (kv_dtype == KANSO_KV_F32) {
            const float* src = static_cast<const float*>(pool) + row_idx * d;
            std::memcpy(out, src, d * sizeof(float));
        } else if (kv_dtype == KANSO_KV_INT8) {
            // read_quantized_kv_token / gather_dequantized_blocks, INT8 arm
            // (src/kv_cache/quantized_storage.rs:351-358): (q as f32) * scale.
            const int8_t* src = static_cast<const int8_t*>(pool) + row_idx * d;
            const float sc = static_cast<const float*>(scales)[row_idx];
            for (uint32_t i = 0; i < d; ++i) out[i] = static_cast<float>(src[i]) * sc;
        } else if (kv_dtype == KANSO_KV_FP8) {
            // FP8 arm (quantized_storage.rs:351-358, fp8_to_f32 :438-449): the E4M3
            // value of the byte times the row's scale.
            const uint8_t* src = static_cast<const uint8_t*>(pool) + row_idx * d;
            const float sc = static_cast<const float*>(scales)[row_idx];
            for (uint32_t i = 0; i < d; ++i) out[i] = oracle_e4m3_to_f32(src[i]) * sc;
        } else {
            // BlockQ8_0::dequantize (src/quant/q8_0.rs:35-39): d * (q as f32), with d
            // read back from its f16 storage.
            const int8_t* src = static_cast<const int8_t*>(pool) + row_idx * d;
            const uint16_t* sc = static_cast<const uint16_t*>(scales) + row_idx * (d / 32);
            for (uint32_t i = 0; i < d; ++i)
                out[i] = oracle_f16_to_f32(sc[i / 32]) * static_cast<float>(src[i]);
        }
    }
};

// One query row against keys [0, limit) of an already gathered context
// ([ctx][d] rows of this KV head). Arithmetic of cpu_paged_attention
// (src/metal/paged_attention.rs:122-173).
void attend_row(const float* qv, const float* kctx, const float* vctx, uint32_t limit,
                uint32_t d, float scale, float* out, std::vector<float>& scores) {
    scores.resize(limit);
    for (uint32_t t = 0; t < limit; ++t) {
        float dot = 0.0f;
        const float* kr = kctx + static_cast<size_t>(t) * d;
        for (uint32_t i = 0; i < d; ++i) dot += qv[i] * kr[i];
        scores[t] = dot * scale;
    }
    float max_score = -INFINITY;
    for (uint32_t t = 0; t < limit; ++t)
        if (scores[t] > max_score) max_score = scores[t];
    float sum_exp = 0.0f;
    for (uint32_t t = 0; t < limit; ++t) {
        const float ex = std::exp(scores[t] - max_score);
        scores[t] = ex;
        sum_exp += ex;
    }
    const float inv_sum = sum_exp > 0.0f ? 1.0f / sum_exp : 0.0f;
    for (uint32_t i = 0; i < d; ++i) out[i] = 0.0f;
    for (uint32_t t = 0; t < limit; ++t) {
        const float w = scores[t] * inv_sum;
        const float* vr = vctx + static_cast<size_t>(t) * d;
        for (uint32_t i = 0; i < d; ++i) out[i] += w * vr[i];
    }
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------- attention

void oracle_paged_attention(const float* q, const float* k_cache, const float* v_cache,
                            const uint32_t* block_tables, const uint32_t* context_lens,
                            const kanso_paged_attention_params* p, float* out) {
    // src/metal/paged_attention.rs:84-178, loop for loop.
    const size_t num_seqs = p->num_seqs, num_heads = p->num_heads;
    const size_t num_kv_heads = p->num_kv_heads, head_dim = p->head_dim;
    const size_t block_size = p->block_size, max_num_blocks = p->max_num_blocks_per_seq;
    const float scale = p->scale;
    const size_t kv_group_size = num_heads / num_kv_heads;
    std::fill(out, out + num_seqs * num_heads * head_dim, 0.0f);
    std::vector<float> scores, exp_scores;
    for (size_t s = 0; s < num_seqs; ++s) {
        const size_t ctx_len = context_lens[s];
        if (ctx_len == 0) continue;
        for (size_t h = 0; h < num_heads; ++h) {
            const size_t kv_h = h / kv_group_size;
            const float* q_vec = q + (s * num_heads + h) * head_dim;
            scores.clear();
            for (size_t t = 0; t < ctx_len; ++t) {
                const size_t b_idx = t / block_size, b_off = t % block_size;
                const size_t phys = block_tables[s * max_num_blocks + b_idx];
                const size_t k_off = phys * (block_size * num_kv_heads * head_dim) +
                                     b_off * (num_kv_heads * head_dim) + kv_h * head_dim;
                float dot = 0.0f;
                for (size_t d = 0; d < head_dim; ++d) dot += q_vec[d] * k_cache[k_off + d];
                scores.push_back(dot * scale);
            }
            float max_score = -INFINITY;
            for (float sc : scores)
                if (sc > max_score) max_score = sc;
            float sum_exp = 0.0f;
            exp_scores.clear();
            for (float sc : scores) {
                const float ex = std::exp(sc - max_score);
                exp_scores.push_back(ex);
                sum_exp += ex;
            }
            const float inv_sum = sum_exp > 0.0f ? 1.0f / sum_exp : 0.0f;
            float* o = out + (s * num_heads + h) * head_dim;
            for (size_t t = 0; t < ctx_len; ++t) {
                const float weight = exp_scores[t] * inv_sum;
                const size_t b_idx = t / block_size, b_off = t % block_size;
                const size_t phys = block_tables[s * max_num_blocks + b_idx];
                const size_t v_off = phys * (block_size * num_kv_heads * head_dim) +
                                     b_off * (num_kv_heads * head_dim) + kv_h * head_dim;
                for (size_t d = 0; d < head_dim; ++d) o[d] += weight * v_cache[v_off + d];
            }
        }
    }
}

int oracle_ragged_attention(const float* q, const void* k_pool, const void* v_pool,
                            const void* k_scales, const void* v_scales,
                            const uint32_t* block_tables, const int32_t* cu_seqlens,
                            const uint32_t* context_lens,
                            const kanso_ragged_attention_params* p, float* out,
                            int nthreads) {
    const uint32_t S = p->num_seqs, H = p->num_heads, HKV = p->num_kv_heads;
    const uint32_t D = p->head_dim, BS = p->block_size, MB = p->max_num_blocks_per_seq;
    if (HKV == 0 || H % HKV != 0) return -1;
    const uint32_t G = H / HKV;
    // Shape checks of forward_batch_rows (src/model.rs:1485-1493) and the capacity /
    // empty-context rejections of gpu_paged_attention_v2 (paged_attention.rs:342-355).
    for (uint32_t s = 0; s < S; ++s) {
        const int32_t ql = cu_seqlens[s + 1] - cu_seqlens[s];
        const uint32_t ctx = context_lens[s];
        if (ql <= 0 || ctx == 0 || static_cast<uint32_t>(ql) > ctx || ctx > MB * BS) return -1;
        for (uint32_t b = 0; b < (ctx + BS - 1) / BS; ++b)
            if (block_tables[static_cast<size_t>(s) * MB + b] >= p->num_blocks) return -1;
    }
    const DequantView kv{p->kv_dtype, BS, HKV, D, k_pool, k_scales};
    const DequantView vv{p->kv_dtype, BS, HKV, D, v_pool, v_scales};
    const int64_t units = static_cast<int64_t>(S) * HKV;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1)
    for (int64_t u = 0; u < units; ++u) {
        const uint32_t s = static_cast<uint32_t>(u / HKV), kvh = static_cast<uint32_t>(u % HKV);
        const uint32_t ctx = context_lens[s];
        const uint32_t ql = static_cast<uint32_t>(cu_seqlens[s + 1] - cu_seqlens[s]);
        const uint32_t start = ctx - ql;
        // gather_blocks (src/kv_cache/storage.rs:283-335 / quantized_storage.rs:284-383).
        std::vector<float> kctx(static_cast<size_t>(ctx) * D), vctx(static_cast<size_t>(ctx) * D);
        for (uint32_t t = 0; t < ctx; ++t) {
            const uint32_t phys = block_tables[static_cast<size_t>(s) * MB + t / BS];
            kv.row(phys, t % BS, kvh, &kctx[static_cast<size_t>(t) * D]);
            vv.row(phys, t % BS, kvh, &vctx[static_cast<size_t>(t) * D]);
        }
        std::vector<float> scores;
        for (uint32_t g = 0; g < G; ++g) {
            const uint32_t h = kvh * G + g;  // head = kv_head * group + g (model.rs:1800-1802)
            for (uint32_t i = 0; i < ql; ++i) {
                const size_t row = static_cast<size_t>(cu_seqlens[s]) + i;
                // Row i may attend keys 0..=start+i (model.rs:1513-1518).
                attend_row(q + (row * H + h) * D, kctx.data(), vctx.data(), start + i + 1, D,
                           p->scale, out + (row * H + h) * D, scores);
            }
        }
    }
    return 0;
}

// ---------------------------------------------------------------- packing

int oracle_pack_step(const kanso_seq_plan* plan, uint32_t num_seqs,
                     const uint32_t* token_arena, const uint32_t* table_arena,
                     uint32_t block_size, int32_t* cu_seqlens, int32_t* seq_of_query,
                     int32_t* positions, int64_t* slot_mapping, uint32_t* tokens,
                     uint32_t* block_tables, uint32_t* context_lens,
                     uint32_t* max_blocks_out) {
    // Engine::step packing (src/engine.rs:376-402).
    uint32_t n = 0;
    cu_seqlens[0] = 0;
    for (uint32_t s = 0; s < num_seqs; ++s) {
        const kanso_seq_plan& pl = plan[s];
        const uint32_t* table = table_arena + pl.table_offset;
        for (uint32_t i = 0; i < pl.q_len; ++i) {
            const uint32_t pos = pl.start_pos + i;
            const uint32_t block_idx = pos / block_size;
            if (block_idx >= pl.table_len) return -1;  // engine.rs:387-394
            tokens[n] = token_arena[pl.token_offset + pos];
            positions[n] = static_cast<int32_t>(pos);
            slot_mapping[n] = static_cast<int64_t>(table[block_idx]) * block_size + pos % block_size;
            seq_of_query[n] = static_cast<int32_t>(s);
            ++n;
        }
        context_lens[s] = pl.start_pos + pl.q_len;
        cu_seqlens[s + 1] = static_cast<int32_t>(n);
    }
    // PaddedDecodeTables::new (src/model.rs:84-105).
    uint32_t max_blocks = 1;
    for (uint32_t s = 0; s < num_seqs; ++s)
        max_blocks = std::max(max_blocks, std::max((context_lens[s] + block_size - 1) / block_size, 1u));
    for (uint32_t s = 0; s < num_seqs; ++s) {
        const uint32_t needed = std::max((context_lens[s] + block_size - 1) / block_size, 1u);
        if (plan[s].table_len < needed) return -1;  // model.rs:92-100
        for (uint32_t b = 0; b < max_blocks; ++b)
            block_tables[static_cast<size_t>(s) * max_blocks + b] =
                table_arena[plan[s].table_offset + std::min(b, needed - 1)];
    }
    *max_blocks_out = max_blocks;
    return 0;
}

// ---------------------------------------------------------------- quantization

float oracle_quantize_head_int8(const float* x, uint32_t n, int8_t* q) {
    // quantize_head_slice, QuantMode::Int8 (src/kv_cache/quantized_storage.rs:452-469).
    float amax = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        const float ax = std::fabs(x[i]);
        if (ax > amax) amax = ax;
    }
    const float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv_scale = 1.0f / scale;
    for (uint32_t i = 0; i < n; ++i) q[i] = clamp_i8(rust_round(x[i] * inv_scale), -127.0f, 127.0f);
    return scale;
}

// OCP FP8 E4M3FN (float8 0.7.0's F8E4M3, called at quantized_storage.rs:444 and
// :480; the crate is not vendored): sign, 4 exponent bits with bias 7, 3 mantissa
// bits, subnormals of 2^-9 steps, no infinities, NaN = S.1111.111, largest finite
// 448. Encoding rounds to nearest, ties to even (IEEE's default); inputs of 464
// and above saturate to 448 (the KV quantizer never produces them: |x / scale| <= 64).
uint8_t oracle_f32_to_e4m3(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    const uint8_t sign = static_cast<uint8_t>((u >> 24) & 0x80u);
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7f;  // NaN
    if (a >= 0x43e80000u) return sign | 0x7e;  // >= 464
    if (a >= 0x3c800000u) {                    // >= 2^-6: normal
        const uint32_t r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;  // 3 mantissa bits, RNE
        return static_cast<uint8_t>(sign | (r - (120u << 3)));
    }
    float f;
    std::memcpy(&f, &a, 4);
    return static_cast<uint8_t>(sign | static_cast<uint8_t>(std::nearbyint(f * 512.0f)));  // m * 2^-9
}

float oracle_e4m3_to_f32(uint8_t b) {
    const uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
    float v;
    if ((b & 0x7f) == 0x7f) {
        v = std::nanf("");
    } else if (e == 0) {
        v = static_cast<float>(m) * 0.001953125f;
    } else {
        const uint32_t bits = ((e + 120u) << 23) | (m << 20);
        std::memcpy(&v, &bits, 4);
    }
    return (b & 0x80) ? -v : v;
}

float oracle_quantize_head_fp8(const float* x, uint32_t n, uint8_t* q) {
    // quantize_head_slice, QuantMode::Fp8 (src/kv_cache/quantized_storage.rs:470-486):
    // scale = 2^ceil(log2(amax / 64)) (1 for amax = 0), q = E4M3(x * (1 / scale)).
    // ceil(log2 y) is taken exactly from y's exponent bits; the reference's f32
    // log2 could round to an integer for y within an ulp above a power of two,
    // where the two differ (parity unpinned there).
    float amax = 0.0f;
    for (uint32_t i = 0; i < n; ++i) {
        const float ax = std::fabs(x[i]);
        if (ax > amax) amax = ax;
    }
    float scale = 1.0f;
    if (amax > 0.0f) {
        int e2;
        const float fr = std::frexp(amax / 64.0f, &e2);  // amax/64 = fr * 2^e2, fr in [0.5, 1)
        const int k = fr == 0.5f ? e2 - 1 : e2;
        scale = std::ldexp(1.0f, k);
    }
    const float inv_scale = 1.0f / scale;
    for (uint32_t i = 0; i < n; ++i) q[i] = oracle_f32_to_e4m3(x[i] * inv_scale);
    return scale;
}

float oracle_quantize_q8_0_block(const float* x, int8_t* qs) {
    // BlockQ8_0::from_f32_slice (src/quant/q8_0.rs:13-32).
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        const float ax = std::fabs(x[i]);
        if (ax > amax) amax = ax;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    for (int i = 0; i < 32; ++i) qs[i] = clamp_i8(rust_round(x[i] * id), -128.0f, 127.0f);
    return d;
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xffu;
    const uint32_t mant = x & 0x7fffffu;
    if (exp == 0xffu) return static_cast<uint16_t>(sign | 0x7c00u | (mant ? 0x200u | (mant >> 13) : 0u));
    const int e = static_cast<int>(exp) - 127 + 15;
    if (e >= 0x1f) return static_cast<uint16_t>(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return static_cast<uint16_t>(sign);
        const uint32_t m = mant | 0x800000u;
        const int shift = 14 - e;
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) ++h;
        return static_cast<uint16_t>(sign | h);
    }
    uint32_t h = (static_cast<uint32_t>(e) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // a carry rolls into the exponent
    return static_cast<uint16_t>(sign | h);
}

float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (static_cast<uint32_t>(h) & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t mant = h & 0x3ffu;
    uint32_t x;
    if (exp == 0) {
        if (mant == 0) {
            x = sign;
        } else {  // subnormal: mant * 2^-24, exact in f32
            float v = static_cast<float>(mant) * 5.9604644775390625e-08f;
            std::memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (exp == 0x1fu) {
        x = sign | 0x7f800000u | (mant << 13);
    } else {
        x = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

int oracle_kv_append(uint32_t kv_dtype, const float* k, const float* v,
                     const int64_t* slot_mapping, uint32_t num_tokens, uint32_t num_blocks,
                     uint32_t block_size, uint32_t num_kv_heads, uint32_t head_dim,
                     void* k_pool, void* v_pool, void* k_scales, void* v_scales) {
    // KvSlotPlan::new bounds check (src/kv_cache/kind.rs:129-137).
    const int64_t num_slots = static_cast<int64_t>(num_blocks) * block_size;
    for (uint32_t t = 0; t < num_tokens; ++t)
        if (slot_mapping[t] < 0 || slot_mapping[t] >= num_slots) return -1;
    if (kv_dtype == KANSO_KV_Q8_0 && head_dim % 32 != 0) return -1;
    const size_t row = static_cast<size_t>(num_kv_heads) * head_dim;
    for (uint32_t t = 0; t < num_tokens; ++t) {
        const size_t slot = static_cast<size_t>(slot_mapping[t]);  // = block * bs + offset
        const float* kr = k + t * row;
        const float* vr = v + t * row;
        if (kv_dtype == KANSO_KV_F32) {
            // KvStorage::write_kv_slots: scatter of the [Hkv, D] row (storage.rs:219-254).
            std::memcpy(static_cast<float*>(k_pool) + slot * row, kr, row * sizeof(float));
            std::memcpy(static_cast<float*>(v_pool) + slot * row, vr, row * sizeof(float));
        } else if (kv_dtype == KANSO_KV_INT8) {
            // write_quantized_kv_token (quantized_storage.rs:187-201): per KV head,
            // scale_idx = offset * n_kv_heads + h inside the block.
            for (uint32_t h = 0; h < num_kv_heads; ++h) {
                const size_t r = slot * num_kv_heads + h;
                static_cast<float*>(k_scales)[r] = oracle_quantize_head_int8(
                    kr + h * head_dim, head_dim, static_cast<int8_t*>(k_pool) + r * head_dim);
                static_cast<float*>(v_scales)[r] = oracle_quantize_head_int8(
                    vr + h * head_dim, head_dim, static_cast<int8_t*>(v_pool) + r * head_dim);
            }
        } else if (kv_dtype == KANSO_KV_FP8) {
            // write_quantized_kv_token, Fp8 mode: the INT8 layout with E4M3 bytes.
            for (uint32_t h = 0; h < num_kv_heads; ++h) {
                const size_t r = slot * num_kv_heads + h;
                static_cast<float*>(k_scales)[r] = oracle_quantize_head_fp8(
                    kr + h * head_dim, head_dim, static_cast<uint8_t*>(k_pool) + r * head_dim);
                static_cast<float*>(v_scales)[r] = oracle_quantize_head_fp8(
                    vr + h * head_dim, head_dim, static_cast<uint8_t*>(v_pool) + r * head_dim);
            }
        } else {
            // Q8_0 rows: BlockQ8_0::from_f32_slice per 32 elements, d stored as f16.
            for (uint32_t h = 0; h < num_kv_heads; ++h) {
                const size_t r = slot * num_kv_heads + h;
                for (uint32_t b = 0; b < head_dim / 32; ++b) {
                    const float dk = oracle_quantize_q8_0_block(
                        kr + h * head_dim + b * 32, static_cast<int8_t*>(k_pool) + r * head_dim + b * 32);
                    const float dv = oracle_quantize_q8_0_block(
                        vr + h * head_dim + b * 32, static_cast<int8_t*>(v_pool) + r * head_dim + b * 32);
                    static_cast<uint16_t*>(k_scales)[r * (head_dim / 32) + b] = oracle_f32_to_f16(dk);
                    static_cast<uint16_t*>(v_scales)[r * (head_dim / 32) + b] = oracle_f32_to_f16(dv);
                }
            }
        }
    }
    return 0;
}

// ---------------------------------------------------------------- GEMV

namespace {
struct Q8Block16 { uint16_t d; int8_t qs[32]; };           // GGUF block_q8_0, 34 B
struct Q8Block32 { float d; int8_t qs[32]; };              // src/quant/q8_0.rs:4-9, 36 B
struct Q4KBlock16 { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; };  // 144 B
struct Q4KBlock32 { float d, dmin; uint8_t scales[12]; uint8_t qs[128]; };     // 148 B
static_assert(sizeof(Q8Block16) == 34, "block_q8_0");
static_assert(sizeof(Q8Block32) == 36, "BlockQ8_0");
static_assert(sizeof(Q4KBlock16) == 144, "block_q4_K");
static_assert(sizeof(Q4KBlock32) == 148, "BlockQ4_K");

// scalar_dot_q8_0 (src/quant/q8_0.rs:51-57).
inline float dot_q8(float d, const int8_t* qs, const float* x) {
    float sum = 0.0f;
    for (int i = 0; i < 32; ++i) sum += static_cast<float>(qs[i]) * x[i];
    return d * sum;
}

void dequant_q4k(float d, float dmin, const uint8_t* scales, const uint8_t* qs, float* out) {
    // BlockQ4_K::dequantize (src/quant/q4_k.rs:30-55).
    uint32_t is = 0, y = 0;
    for (uint32_t j = 0; j < 256; j += 64) {
        const uint8_t* q_sub = qs + j / 2;
        uint8_t sc1, m1, sc2, m2;
        oracle_get_scale_min_k4(is, scales, &sc1, &m1);
        const float d1 = d * static_cast<float>(sc1), min1 = dmin * static_cast<float>(m1);
        oracle_get_scale_min_k4(is + 1, scales, &sc2, &m2);
        const float d2 = d * static_cast<float>(sc2), min2 = dmin * static_cast<float>(m2);
        for (int l = 0; l < 32; ++l) out[y++] = d1 * static_cast<float>(q_sub[l] & 0xF) - min1;
        for (int l = 0; l < 32; ++l) out[y++] = d2 * static_cast<float>(q_sub[l] >> 4) - min2;
        is += 2;
    }
}

// scalar_dot_q4_k (src/quant/q4_k.rs:150-159).
inline float dot_q4k(const float* deq, const float* x) {
    float sum = 0.0f;
    for (int i = 0; i < 256; ++i) sum += deq[i] * x[i];
    return sum;
}
}  // namespace

void oracle_get_scale_min_k4(uint32_t j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    // src/quant/q4_k.rs:16-26.
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = static_cast<uint8_t>((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = static_cast<uint8_t>((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

void oracle_gemv_q8_0(const void* w, const float* x, float* y, uint32_t rows, uint32_t cols,
                      uint32_t batch, int nthreads) {
    // scalar_gemv_q8_0 (src/quant/q8_0.rs:69-93), one GEMV per activation row.
    const uint32_t bpr = cols / 32;
    const Q8Block16* wb = static_cast<const Q8Block16*>(w);
    const int64_t total = static_cast<int64_t>(batch) * rows;
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
    for (int64_t br = 0; br < total; ++br) {
        const uint32_t b = static_cast<uint32_t>(br / rows), r = static_cast<uint32_t>(br % rows);
        const float* xb = x + static_cast<size_t>(b) * cols;
        float sum = 0.0f;
        for (uint32_t k = 0; k < bpr; ++k) {
            const Q8Block16& blk = wb[static_cast<size_t>(r) * bpr + k];
            sum += dot_q8(oracle_f16_to_f32(blk.d), blk.qs, xb + k * 32);
        }
        y[static_cast<size_t>(b) * rows + r] = sum;
    }
}

void oracle_gemv_q8_0_f32d(const void* w, const float* x, float* y, uint32_t rows,
                           uint32_t cols, uint32_t batch) {
    const uint32_t bpr = cols / 32;
    const Q8Block32* wb = static_cast<const Q8Block32*>(w);
    for (uint32_t b = 0; b < batch; ++b)
        for (uint32_t r = 0; r < rows; ++r) {
            float sum = 0.0f;
            for (uint32_t k = 0; k < bpr; ++k) {
                const Q8Block32& blk = wb[static_cast<size_t>(r) * bpr + k];
                sum += dot_q8(blk.d, blk.qs, x + static_cast<size_t>(b) * cols + k * 32);
            }
            y[static_cast<size_t>(b) * rows + r] = sum;
        }
}

void oracle_dequant_q4_k(const void* blk, float* out256) {
    const Q4KBlock16* b = static_cast<const Q4KBlock16*>(blk);
    dequant_q4k(oracle_f16_to_f32(b->d), oracle_f16_to_f32(b->dmin), b->scales, b->qs, out256);
}

void oracle_dequant_q4_k_f32d(const void* blk, float* out256) {
    const Q4KBlock32* b = static_cast<const Q4KBlock32*>(blk);
    dequant_q4k(b->d, b->dmin, b->scales, b->qs, out256);
}

void oracle_gemv_q4_k(const void* w, const float* x, float* y, uint32_t rows, uint32_t cols,
                      uint32_t batch, int nthreads) {
    // scalar_gemv_q4_k (src/quant/q4_k.rs:162-186).
    const uint32_t bpr = cols / 256;
    const Q4KBlock16* wb = static_cast<const Q4KBlock16*>(w);
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
    for (int64_t r = 0; r < static_cast<int64_t>(rows); ++r) {
        float deq[256];
        std::vector<float> sums(batch, 0.0f);
        for (uint32_t k = 0; k < bpr; ++k) {
            oracle_dequant_q4_k(&wb[static_cast<size_t>(r) * bpr + k], deq);
            for (uint32_t b = 0; b < batch; ++b)
                sums[b] += dot_q4k(deq, x + static_cast<size_t>(b) * cols + k * 256);
        }
        for (uint32_t b = 0; b < batch; ++b) y[static_cast<size_t>(b) * rows + r] = sums[b];
    }
}

void oracle_gemv_q4_k_f32d(const void* w, const float* x, float* y, uint32_t rows,
                           uint32_t cols, uint32_t batch) {
    const uint32_t bpr = cols / 256;
    const Q4KBlock32* wb = static_cast<const Q4KBlock32*>(w);
    float deq[256];
    for (uint32_t b = 0; b < batch; ++b)
        for (uint32_t r = 0; r < rows; ++r) {
            float sum = 0.0f;
            for (uint32_t k = 0; k < bpr; ++k) {
                oracle_dequant_q4_k_f32d(&wb[static_cast<size_t>(r) * bpr + k], deq);
                sum += dot_q4k(deq, x + static_cast<size_t>(b) * cols + k * 256);
            }
            y[static_cast<size_t>(b) * rows + r] = sum;
        }
}

void oracle_dequant_row_q8_0(const void* blocks, uint32_t n, float* out) {
    // BlockQ8_0::dequantize (src/quant/q8_0.rs:35-39): d * q per element.
    const Q8Block16* b = static_cast<const Q8Block16*>(blocks);
    for (uint32_t i = 0; i < n; ++i) {
        const Q8Block16& blk = b[i / 32];
        out[i] = oracle_f16_to_f32(blk.d) * static_cast<float>(blk.qs[i % 32]);
    }
}

void oracle_quantize_row_q8_0(const float* x, uint32_t n, void* blocks) {
    Q8Block16* out = static_cast<Q8Block16*>(blocks);
    for (uint32_t b = 0; b < n / 32; ++b) {
        const float d = oracle_quantize_q8_0_block(x + b * 32, out[b].qs);
        out[b].d = oracle_f32_to_f16(d);
    }
}

void oracle_quantize_row_q4_k(const float* x, uint32_t n, void* blocks) {
    // This build's own Q4_K quantizer (the reference has none; see the header).
    Q4KBlock16* out = static_cast<Q4KBlock16*>(blocks);
    for (uint32_t sb = 0; sb < n / 256; ++sb) {
        const float* xs = x + sb * 256;
        float scale[8], minv[8];
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; ++j) {
            float lo = xs[j * 32], hi = xs[j * 32];
            for (int l = 1; l < 32; ++l) {
                lo = std::min(lo, xs[j * 32 + l]);
                hi = std::max(hi, xs[j * 32 + l]);
            }
            lo = std::min(lo, 0.0f);  // the stored min is subtracted: w = d*sc*q - dmin*m
            scale[j] = (hi - lo) / 15.0f;
            minv[j] = -lo;
            max_scale = std::max(max_scale, scale[j]);
            max_min = std::max(max_min, minv[j]);
        }
        const float d = max_scale / 63.0f, dmin = max_min / 63.0f;
        const uint16_t d16 = oracle_f32_to_f16(d), dmin16 = oracle_f32_to_f16(dmin);
        const float df = oracle_f16_to_f32(d16), dminf = oracle_f16_to_f32(dmin16);
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 8; ++j) {
            sc[j] = static_cast<uint8_t>(std::min(63.0f, df > 0.0f ? std::round(scale[j] / df) : 0.0f));
            mn[j] = static_cast<uint8_t>(std::min(63.0f, dminf > 0.0f ? std::round(minv[j] / dminf) : 0.0f));
        }
        Q4KBlock16& blk = out[sb];
        blk.d = d16;
        blk.dmin = dmin16;
        for (int j = 0; j < 4; ++j) {
            blk.scales[j] = static_cast<uint8_t>((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            blk.scales[j + 4] = static_cast<uint8_t>((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
            blk.scales[j + 8] = static_cast<uint8_t>((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
        }
        for (int j = 0; j < 8; ++j) {
            const float ds = df * static_cast<float>(sc[j]);
            const float dm = dminf * static_cast<float>(mn[j]);
            for (int l = 0; l < 32; ++l) {
                const float v = ds > 0.0f ? std::round((xs[j * 32 + l] + dm) / ds) : 0.0f;
                const uint8_t nib = static_cast<uint8_t>(std::min(15.0f, std::max(0.0f, v)));
                uint8_t& byte = blk.qs[(j / 2) * 32 + l];
                if (j % 2 == 0) byte = static_cast<uint8_t>((byte & 0xF0) | nib);
                else byte = static_cast<uint8_t>((byte & 0x0F) | (nib << 4));
            }
        }
    }
}

// ---------------------------------------------------------------- decoder glue

void oracle_rmsnorm(const float* x, const float* w, float* y, uint32_t rows, uint32_t n,
                    float eps) {
    for (uint32_t r = 0; r < rows; ++r) {
        const float* xr = x + static_cast<size_t>(r) * n;
        float sq = 0.0f;
        for (uint32_t i = 0; i < n; ++i) sq += xr[i] * xr[i];
        const float rms = std::sqrt(sq / static_cast<float>(n) + eps);
        for (uint32_t i = 0; i < n; ++i) y[static_cast<size_t>(r) * n + i] = xr[i] / rms * w[i];
    }
}

void oracle_rope_table(uint32_t len, uint32_t head_dim, float theta, float* cos_t,
                       float* sin_t) {
    const uint32_t half = head_dim / 2;
    std::vector<float> th(half);
    for (uint32_t j = 0; j < half; ++j)
        th[j] = std::pow(theta, -2.0f * static_cast<float>(j) / static_cast<float>(head_dim));
    for (uint32_t p = 0; p < len; ++p)
        for (uint32_t j = 0; j < half; ++j) {
            const float a = static_cast<float>(p) * th[j];
            cos_t[static_cast<size_t>(p) * half + j] = std::cos(a);
            sin_t[static_cast<size_t>(p) * half + j] = std::sin(a);
        }
}

void oracle_rope_apply(float* x, uint32_t rows, uint32_t heads, uint32_t head_dim,
                       const int32_t* positions, const float* cos_t, const float* sin_t) {
    const uint32_t half = head_dim / 2;
    for (uint32_t r = 0; r < rows; ++r) {
        const float* c = cos_t + static_cast<size_t>(positions[r]) * half;
        const float* s = sin_t + static_cast<size_t>(positions[r]) * half;
        for (uint32_t h = 0; h < heads; ++h) {
            float* v = x + (static_cast<size_t>(r) * heads + h) * head_dim;
            for (uint32_t j = 0; j < half; ++j) {
                const float x1 = v[j], x2 = v[j + half];
                const float a = x1 * c[j], b = x2 * s[j];
                const float e = x1 * s[j], f = x2 * c[j];
                v[j] = a - b;
                v[j + half] = e + f;
            }
        }
    }
}

void oracle_silu_mul(const float* gate, const float* up, float* y, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) {
        const float g = gate[i];
        y[i] = g / (1.0f + std::exp(-g)) * up[i];
    }
}

uint32_t oracle_greedy(const float* logits, uint32_t n) {
    uint32_t best = 0;
    float best_val = -INFINITY;
    for (uint32_t i = 0; i < n; ++i)
        if (logits[i] > best_val) {
            best_val = logits[i];
            best = i;
        }
    return best;
}

uint64_t oracle_fnv1a_64(const uint32_t* tokens, size_t n) {
    uint64_t hash = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < n; ++i) hash = (hash ^ static_cast<uint64_t>(tokens[i])) * 0x100000001b3ull;
    return hash;
}

}  // extern "C"

// ---------------------------------------------------------------- host bandwidth

double oracle_stream_triad(uint64_t n, int nthreads, int reps) {
    std::vector<double> a(n), b(n), c(n);
    const double s = 3.0;
    const int64_t N = static_cast<int64_t>(n);
#ifdef _OPENMP
#pragma omp parallel for num_threads(nthreads) schedule(static)
#endif
    for (int64_t i = 0; i < N; ++i) {
        a[i] = 0.0;
        b[i] = 1.0;
        c[i] = 2.0;
    }
    double best = 0.0;
    for (int r = 0; r < reps; ++r) {
#ifdef _OPENMP
        const double t0 = omp_get_wtime();
#pragma omp parallel for num_threads(nthreads) schedule(static)
        for (int64_t i = 0; i < N; ++i) a[i] = b[i] + s * c[i];
        const double t = omp_get_wtime() - t0;
#else
        (void)nthreads;
        const double t = 1.0;
#endif
        best = std::max(best, 24.0 * static_cast<double>(n) / t / 1e9);
    }
    volatile double sink = a[n / 2];  // the stores stay observable
    (void)sink;
    return best;
}
