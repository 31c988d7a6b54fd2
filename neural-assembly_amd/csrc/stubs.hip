// stubs.hip -- entry points of the reference's C ABI outside this library's
// scope (the reference's pyneural/core.py binds all of them at import; the
// header lists which binding each one answers).  They touch no device and
// allocate nothing: an error code, NULL, 0 or NaN, with
// NEURAL_ERR_NOT_IMPLEMENTED recorded as the thread's last error.
#include <cstdint>
#include <limits>

#include "common.hpp"

extern "C" {

int attention_scaled_dot_product(void *, void *, void *, void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int batchnorm1d_backward(void *, void *, void *, void *, void *, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int batchnorm1d_forward(void *, void *, void *, int64_t, int) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t batchnorm1d_num_features(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
void *batchnorm1d_beta(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void *batchnorm1d_create(int64_t, double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void *batchnorm1d_gamma(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void *batchnorm1d_running_mean(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void *batchnorm1d_running_var(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void batchnorm1d_free(void *) { }
int conv2d_layer_backward(void *, void *, void *, int64_t, int64_t, int64_t, void *, void *, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int conv2d_layer_forward(void *, void *, int64_t, int64_t, int64_t, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t conv2d_layer_in_channels(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t conv2d_layer_kernel_h(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t conv2d_layer_kernel_w(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t conv2d_layer_out_channels(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t conv2d_layer_out_h(void *, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t conv2d_layer_out_w(void *, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t conv2d_layer_padding(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t conv2d_layer_stride(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t conv2d_layer_weight_size(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t conv2d_output_size(int64_t, int64_t, int64_t, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
void *conv2d_layer_bias(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void *conv2d_layer_create(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void *conv2d_layer_weight(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void conv2d_layer_free(void *) { }
int embedding_backward(void *, void *, int64_t, void *, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int embedding_forward(void *, void *, int64_t, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t embedding_dim(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t embedding_num_embeddings(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
void *embedding_create(int64_t, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void *embedding_weight(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void embedding_free(void *) { }
double fuzzy_and(double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double fuzzy_defuzz_bisector(void *, void *, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double fuzzy_defuzz_centroid(void *, void *, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double fuzzy_defuzz_mom(void *, void *, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double fuzzy_gaussian(double, double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double fuzzy_not(double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double fuzzy_or(double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double fuzzy_trapezoidal(double, double, double, double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double fuzzy_triangular(double, double, double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
int fuzzy_system_add_input_mf(void *, int, int, double, double, double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int fuzzy_system_add_output_mf(void *, int, double, double, double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int fuzzy_system_add_rule(void *, void *, void *, int, int, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int fuzzy_system_defuzz_method(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int fuzzy_system_evaluate(void *, void *, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int fuzzy_system_n_inputs(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int fuzzy_system_n_rules(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int fuzzy_system_resolution(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int fuzzy_system_set_input_range(void *, int, double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int fuzzy_system_set_output_range(void *, double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
void *fuzzy_system_create(int, int, int) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void fuzzy_system_free(void *) { }
double *gru_bias_hh(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
double *gru_bias_ih(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
double *gru_weight_hh(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
double *gru_weight_ih(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
int gru_forward(void *, double *, double *, double *, double *, int64_t, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t gru_hidden_size(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t gru_input_size(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
void *gru_create(int64_t, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void gru_free(void *) { }
int layernorm_backward(void *, void *, void *, void *, void *, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int layernorm_forward(void *, void *, void *, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t layernorm_num_features(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
void *layernorm_beta(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void *layernorm_create(int64_t, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void *layernorm_gamma(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void layernorm_free(void *) { }
double *lstm_bias_hh(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
double *lstm_bias_ih(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
double *lstm_weight_hh(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
double *lstm_weight_ih(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
int lstm_forward(void *, double *, double *, double *, double *, double *, double *, int64_t, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t lstm_hidden_size(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t lstm_input_size(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
void *lstm_create(int64_t, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void lstm_free(void *) { }
const char *neural_get_simd_name(void) {
    return "none (HIP, gfx950)";
}
double compute_sparsity(void *, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double compute_threshold_for_sparsity(void *, int64_t, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
int neural_get_simd_level(void) {
    return 0;  // no host SIMD dispatch: the arithmetic runs on the GPU
}
int neural_matmul(void *, void *, void *) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
int neural_mse_loss(void *, void *, double *) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
int neural_weighted_sample_indices(void *, uint64_t, uint64_t, void *, int) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
int roc_auc_score(void *, void *, int64_t, double *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t count_nonzero(void *, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
void apply_mask(void *, void *, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
void *neural_adam_create(double, double, double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void *neural_adamw_create(double, double, double, double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
double neural_compute_accuracy_from_matrix(void *, int) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double neural_compute_class_f1(void *, int, int) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double neural_compute_class_precision(void *, int, int) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double neural_compute_class_recall(void *, int, int) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
int neural_compute_class_weights(void *, uint64_t, uint64_t, void *) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
int neural_compute_sample_weights(void *, uint64_t, void *, uint64_t, void *) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
void *neural_config_load(const char *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void neural_config_free(void *) { }
int neural_confusion_matrix_update(void *, void *, void *, uint64_t, uint64_t) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
int neural_dataset_get_batch(void *, uint64_t, uint64_t, void **, void **) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
uint64_t neural_dataset_size(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return 0;
}
void *neural_dataset_load_csv(const char *, const char *, uint64_t, uint32_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void neural_dataset_free(void *) { }
int neural_init_he_normal(void *, uint64_t, uint64_t, int) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
int neural_init_he_uniform(void *, uint64_t, uint64_t, int) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
int neural_init_kaiming_uniform(void *, uint64_t, uint64_t, uint64_t, int, int) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
int neural_init_normal_range(void *, uint64_t, float, float, int) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
int neural_init_uniform_range(void *, uint64_t, float, float, int) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
int neural_init_xavier_normal(void *, uint64_t, uint64_t, uint64_t, int) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
int neural_init_xavier_uniform(void *, uint64_t, uint64_t, uint64_t, int) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
int neural_linear_forward(void *, void *, void *) {
    return nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
}
void *neural_linear_bias(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void *neural_linear_create(uint64_t, uint64_t, int) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void *neural_linear_weight(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
void neural_linear_free(void *) { }
double neural_lr_cosine_annealing(double, int, int, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double neural_lr_exponential_decay(double, int, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double neural_lr_step_decay(double, int, int, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
double neural_optimizer_get_lr(void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return std::numeric_limits<double>::quiet_NaN();
}
void neural_optimizer_free(void *) { }
void neural_optimizer_set_lr(void *, double) { }
void *neural_sgd_create(double, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
int avgpool2d_backward(void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int avgpool2d_forward(void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int maxpool2d_backward(void *, void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int maxpool2d_forward(void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t prune_cols(void *, int64_t, int64_t, double, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t prune_magnitude(void *, void *, int64_t, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t prune_rows(void *, int64_t, int64_t, double, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int64_t prune_topk(void *, void *, int64_t, double) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
const char *tb_get_filepath(int) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
const char *tb_get_logdir(int) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return nullptr;
}
int tb_add_histogram_stats(int, const char *, void *, int, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int tb_add_scalar(int, const char *, float, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int tb_add_scalars(int, const char *, void *, void *, int, int64_t) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int tb_close(int) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int tb_create_writer(const char *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int tb_flush(int) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int transformer_block_forward(void *, int64_t, int64_t, int64_t, int64_t, void *, void *, void *, void *, void *, void *, void *, void *, void *, void *, void *, void *, double, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int upsample2d_nearest_backward(void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}
int upsample2d_nearest_forward(void *, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void *) {
    nh::set_error(NEURAL_ERR_NOT_IMPLEMENTED);
    return -1;
}

}  // extern "C"
