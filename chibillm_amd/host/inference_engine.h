// schedule -> build batch -> begin -> execute -> complete, aborting the
// reservation on any failure (src/inference_engine.h:14-78,
// src/inference_engine.cc:153-231).
#pragma once

#include "model_runner.h"

namespace chibillm {

enum class inference_engine_errc : std::uint8_t {
    scheduler_creation_failed,
    sequence_add_failed,
    scheduling_failed,
    model_batch_build_failed,
    model_execution_failed,
    runner_result_count_mismatch,
    batch_abort_failed,
    batch_completion_failed,
    sequence_cancel_failed,
    sequence_remove_failed,
};

[[nodiscard]] inline std::string_view
error_name(inference_engine_errc code) noexcept
{
    static constexpr std::array<std::string_view, 10> names {
        "inference_engine.scheduler_creation_failed",
        "inference_engine.sequence_add_failed",
        "inference_engine.scheduling_failed",
        "inference_engine.model_batch_build_failed",
        "inference_engine.model_execution_failed",
        "inference_engine.runner_result_count_mismatch",
        "inference_engine.batch_abort_failed",
        "inference_engine.batch_completion_failed",
        "inference_engine.sequence_cancel_failed",
        "inference_engine.sequence_remove_failed",
    };
    const auto i = static_cast<std::size_t>(code);
    return i < names.size() ? names[i] : "inference_engine.unknown_error";
}

using inference_engine_error = error<inference_engine_errc>;

class inference_engine {
public:
    [[nodiscard]] static result<inference_engine, inference_engine_error>
    make(scheduler_config config, model_runner& runner);

    inference_engine(inference_engine&&) noexcept = default;
    inference_engine& operator=(inference_engine&&) noexcept = default;

    [[nodiscard]] bool is_finished() const noexcept { return scheduler_.is_finished(); }
    [[nodiscard]] bool has_in_flight_batch() const noexcept
    {
        return scheduler_.has_in_flight_batch();
    }
    [[nodiscard]] const seq* find_sequence(seq_id id) const noexcept
    {
        return scheduler_.find_sequence(id);
    }
    [[nodiscard]] const scheduler& engine_scheduler() const noexcept { return scheduler_; }

    [[nodiscard]] result<void, inference_engine_error> add(seq sequence);
    [[nodiscard]] bool fits_cache(const seq& sequence) const noexcept
    {
        return scheduler_.fits_cache(sequence);
    }
    [[nodiscard]] result<admission_result, inference_engine_error> try_add(seq& sequence);
    [[nodiscard]] result<std::vector<sequence_update>, inference_engine_error> step();
    [[nodiscard]] result<void, inference_engine_error> cancel(seq_id id);
    [[nodiscard]] result<void, inference_engine_error> remove(seq_id id);

    // Host time spent in each stage of the steps so far (no reference
    // counterpart): scheduling, building the model batch, the runner's
    // execute (which includes enqueueing the device work), and completion.
    struct stage_times {
        std::uint64_t steps = 0;
        double schedule_s = 0, build_s = 0, execute_s = 0, complete_s = 0;
    };
    [[nodiscard]] const stage_times& times() const noexcept { return times_; }

private:
    inference_engine(scheduler s, model_runner& runner) noexcept
        : scheduler_(std::move(s))
        , runner_(&runner)
    {}
    result<std::vector<sequence_update>, inference_engine_error>
    run(const scheduled_batch& scheduled);
    failure<inference_engine_error> abandon(const scheduled_batch& batch,
                                            inference_engine_error cause);

    scheduler scheduler_;
    model_runner* runner_;
    stage_times times_;
};

} // namespace chibillm
