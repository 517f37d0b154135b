// The kernel tables (crates/pc-kernels/kernels/inst/instantiate.inc:32-91): one constant-initialised KernelTable per
// ring degree, u32 words, Barrett64 (mm 0). Entries this library does not implement return -1 (argument outside the
// kernel's range), as the reference's table does for an entry a build leaves out.
#include "pc_hip.h"

namespace pch {
#define PCH_DECL(L)                                                  \
    int ntt_fwd_##L(const NttArgs*, pc_stream_t);                    \
    int ntt_inv_##L(const NttArgs*, pc_stream_t);                    \
    int encode_##L(const EncodeArgs*, pc_stream_t);                  \
    int bconv_##L(const BconvArgs*, pc_stream_t);                    \
    int ew_add_##L(const EwArgs*, pc_stream_t);                      \
    int ew_scale_##L(const EwArgs*, pc_stream_t);                    \
    int ew_sub_mul_##L(const EwArgs*, pc_stream_t);                  \
    int ew_copy_##L(const EwArgs*, pc_stream_t);                     \
    int automorph_##L(const AutomorphArgs*, pc_stream_t);            \
    int ks_dot_##L(const KsArgs*, pc_stream_t);                      \
    int ks_dot_key_##L(const KsKeyArgs*, pc_stream_t);               \
    int ksk_expand_##L(const KskExpandArgs*, pc_stream_t);           \
    int ksk_gen_##L(const KskGenArgs*, pc_stream_t);                 \
    int ksk_unpack_##L(const KskUnpackArgs*, pc_stream_t);          \
    int cts_fused_##L(const CtsArgs*, pc_stream_t);                  \
    int cts_fused_regen_##L(const CtsRegenArgs*, pc_stream_t);       \
    int ks_dot_regen_##L(const KsRegenArgs*, pc_stream_t);           \
    int tensor_##L(const TensorArgs*, pc_stream_t);                  \
    int tensor_y_##L(const TensorYArgs*, pc_stream_t);               \
    int tensor_sum_##L(const TensorSumArgs*, pc_stream_t);           \
    int md_epilogue_##L(const MdEpiArgs*, pc_stream_t);              \
    int md_epilogue_to_##L(const MdEpiToArgs*, pc_stream_t);         \
    int wsum_##L(const WsumArgs*, pc_stream_t);                      \
    int wsum_k_##L(const WsumKArgs*, pc_stream_t);                   \
    int wsum_multi_##L(const WsumMultiArgs*, pc_stream_t);           \
    int add_const_##L(const AddConstArgs*, pc_stream_t);             \
    int mul_table_##L(const MulTableArgs*, pc_stream_t);             \
    int mul_add_##L(const MulAddArgs*, pc_stream_t);                 \
    int mul_add_n_##L(const MulAddNArgs*, pc_stream_t);              \
    int rescale_combine_##L(const RescaleCombineArgs*, pc_stream_t); \
    int rescale_combine_to_##L(const RescaleCombineToArgs*, pc_stream_t); \
    int ew_many_##L(const EwManyArgs*, pc_stream_t);                 \
    int submul_many_##L(const SubMulManyArgs*, pc_stream_t);         \
    int rescale_coef_##L(const RescaleArgs*, pc_stream_t);           \
    int spru_fft_pass_##L(const SpruFftArgs*, pc_stream_t);          \
    int spru_scatter_##L(const SpruScatterArgs*, pc_stream_t);       \
    int rescale_fwd_##L(const RescaleNttArgs*, pc_stream_t);         \
    int mod_raise_##L(const ModRaiseArgs*, pc_stream_t);             \
    int small_int_##L(const SmallIntArgs*, pc_stream_t);             \
    int small_int1_##L(const SmallInt1Args*, pc_stream_t);           \
    int encrypt_##L(const EncryptArgs*, pc_stream_t);                \
    int pt_dot_##L(const PtDotArgs*, pc_stream_t);                   \
    int coeff_sum_##L(const CoeffArgs*, pc_stream_t);                \
    int tensor_seeded_##L(const TensorSeededArgs*, pc_stream_t);     \
    int pack_split_##L(const PackSplitArgs*, pc_stream_t);           \
    int pack_dot_##L(const PackDotArgs*, pc_stream_t);               \
    int tensor_multi_##L(const TensorMultiArgs*, pc_stream_t);
PCH_DECL(12)
PCH_DECL(13)
PCH_DECL(14)
PCH_DECL(15)
PCH_DECL(16)

template <class A>
int absent(const A*, pc_stream_t) {
    return -1;
}

#define PCH_TABLE(L)                                                                                                 \
    static const KernelTable TABLE_##L = {                                                                           \
        PC_KERNELS_ABI, 4, 0, L,                                                                                     \
        ntt_fwd_##L, ntt_inv_##L, bconv_##L, ew_add_##L, ew_scale_##L, ew_sub_mul_##L, ew_copy_##L,                  \
        pt_dot_##L, ks_dot_##L, ks_dot_regen_##L, ksk_expand_##L, cts_fused_##L, tensor_##L,                  \
        md_epilogue_##L, wsum_##L, add_const_##L, mul_table_##L, rescale_coef_##L, rescale_combine_##L,            \
        automorph_##L, encode_##L, encrypt_##L, ksk_gen_##L, ksk_unpack_##L, mod_raise_##L,   \
        small_int_##L, absent<SpruExtractArgs>, spru_fft_pass_##L, spru_scatter_##L,                 \
        cts_fused_regen_##L, ks_dot_key_##L, absent<PcmmArgs>, absent<CcmmArgs>, wsum_k_##L, rescale_combine_to_##L, \
        md_epilogue_to_##L, small_int1_##L, coeff_sum_##L, mul_add_##L, rescale_fwd_##L,          \
        mul_add_n_##L, tensor_y_##L, wsum_multi_##L, bconv_##L, absent<TfheArgs>, tensor_sum_##L,                    \
        tensor_multi_##L, tensor_seeded_##L, ew_many_##L, submul_many_##L, pack_split_##L,      \
        pack_dot_##L};
PCH_TABLE(12)
PCH_TABLE(13)
PCH_TABLE(14)
PCH_TABLE(15)
PCH_TABLE(16)
}  // namespace pch

extern "C" const KernelTable* pc_table_u32_barrett64(void) { return &pch::TABLE_16; }

extern "C" const KernelTable* pc_table_u32_logn(uint32_t log_n) {
    switch (log_n) {
        case 12: return &pch::TABLE_12;
        case 13: return &pch::TABLE_13;
        case 14: return &pch::TABLE_14;
        case 15: return &pch::TABLE_15;
        case 16: return &pch::TABLE_16;
        default: return nullptr;
    }
}
