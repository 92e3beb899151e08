// Single-file or sharded safetensors checkpoints (checks and messages of the
// reference's src/io/safetensors_checkpoint.cpp).
#include "qwen3/io/safetensors_checkpoint.h"

#include "json.hpp"
#include "qwen3/io/safetensors_loader.h"

#include <fstream>
#include <limits>
#include <sstream>
#include <stdexcept>

namespace qwen3
{
    namespace
    {
        json::Value read_index(const std::filesystem::path &index_path)
        {
            std::ifstream input{index_path, std::ios::binary};
            if (!input)
                throw std::runtime_error("cannot open checkpoint index: " + index_path.string());
            std::stringstream buffer;
            buffer << input.rdbuf();
            json::Value root;
            try
            {
                root = json::parse(buffer.str());
            }
            catch (const std::runtime_error &e)
            {
                throw std::runtime_error("invalid checkpoint index '" + index_path.string() + "': " + e.what());
            }
            if (root.kind != json::Value::Kind::Object)
                throw std::runtime_error("checkpoint index root must be an object");
            return root;
        }

        std::size_t read_total_size(const json::Value &root)
        {
            const json::Value *meta = root.find("metadata");
            if (meta == nullptr || meta->kind != json::Value::Kind::Object)
                throw std::runtime_error("checkpoint index must contain a metadata object");
            const json::Value *total = meta->find("total_size");
            if (total == nullptr || total->kind != json::Value::Kind::Number || !total->is_unsigned)
                throw std::runtime_error("checkpoint metadata.total_size must be an unsigned integer");
            if (total->unsigned_value > static_cast<std::uint64_t>(std::numeric_limits<std::size_t>::max()))
                throw std::runtime_error("checkpoint total_size is too large");
            return static_cast<std::size_t>(total->unsigned_value);
        }

        std::filesystem::path checked_shard_path(const std::filesystem::path &dir, const std::string &shard)
        {
            if (shard.empty() || shard.find('/') != std::string::npos || shard.find('\\') != std::string::npos)
                throw std::runtime_error("invalid checkpoint shard name: " + shard);
            const std::filesystem::path relative{shard};
            if (relative.is_absolute() || relative.has_parent_path() || relative.extension() != ".safetensors")
                throw std::runtime_error("invalid checkpoint shard name: " + shard);
            const std::filesystem::path full = dir / relative;
            if (!std::filesystem::is_regular_file(full))
                throw std::runtime_error("checkpoint shard does not exist: " + full.string());
            return full;
        }

        std::size_t checked_add(std::size_t a, std::size_t b)
        {
            if (b > std::numeric_limits<std::size_t>::max() - a)
                throw std::overflow_error("checkpoint tensor byte count overflow");
            return a + b;
        }

        bool same_record(const SafetensorsTensorInfo &a, const SafetensorsTensorInfo &b)
        {
            return a.dtype == b.dtype && a.shape == b.shape && a.begin_offset == b.begin_offset &&
                   a.end_offset == b.end_offset;
        }
    } // namespace

    SafetensorsCheckpoint::SafetensorsCheckpoint(const std::filesystem::path &model_directory)
        : model_directory_{std::filesystem::absolute(model_directory)}
    {
        if (!std::filesystem::is_directory(model_directory_))
            throw std::invalid_argument("model directory does not exist: " + model_directory_.string());
        const std::filesystem::path single = model_directory_ / "model.safetensors";
        const std::filesystem::path index = model_directory_ / "model.safetensors.index.json";
        const bool has_single = std::filesystem::is_regular_file(single);
        const bool has_index = std::filesystem::is_regular_file(index);
        if (has_single && has_index)
            throw std::runtime_error("model directory contains both model.safetensors and model.safetensors.index.json");
        if (!has_single && !has_index)
            throw std::runtime_error(
                "model directory contains neither model.safetensors nor model.safetensors.index.json");
        if (has_single)
            open_single_file(single);
        else
            open_sharded_index(index);
    }

    void SafetensorsCheckpoint::open_single_file(const std::filesystem::path &model_path)
    {
        shard_paths_.push_back(model_path);
        SafetensorsLoader loader{model_path};
        for (const auto &entry : loader.metadata().tensors())
            tensors_.emplace(entry.first, TensorLocation{0, entry.second});
        if (tensors_.empty())
            throw std::runtime_error("single-file checkpoint contains no tensors");
    }

    void SafetensorsCheckpoint::open_sharded_index(const std::filesystem::path &index_path)
    {
        const json::Value root = read_index(index_path);
        const std::size_t expected_total = read_total_size(root);
        const json::Value *weight_map = root.find("weight_map");
        if (weight_map == nullptr || weight_map->kind != json::Value::Kind::Object || weight_map->members.empty())
            throw std::runtime_error("checkpoint index weight_map must be a non-empty object");
        std::unordered_map<std::string, std::size_t> shard_by_name;
        std::unordered_map<std::string, std::size_t> expected_shard;
        for (const auto &member : weight_map->members)
        {
            const std::string &tensor_name = member.first;
            if (tensor_name.empty() || member.second.kind != json::Value::Kind::String)
                throw std::runtime_error("checkpoint weight_map contains an invalid entry");
            const std::string &shard = member.second.text;
            auto it = shard_by_name.find(shard);
            std::size_t index = 0;
            if (it == shard_by_name.end())
            {
                index = shard_paths_.size();
                shard_paths_.push_back(checked_shard_path(model_directory_, shard));
                shard_by_name.emplace(shard, index);
            }
            else
            {
                index = it->second;
            }
            expected_shard.insert_or_assign(tensor_name, index); // a repeated key keeps its last value
        }
        std::size_t actual_total = 0;
        for (std::size_t s = 0; s < shard_paths_.size(); ++s)
        {
            SafetensorsLoader loader{shard_paths_[s]};
            for (const auto &entry : loader.metadata().tensors())
            {
                const std::string &name = entry.first;
                actual_total = checked_add(actual_total, entry.second.size_bytes());
                const auto expected = expected_shard.find(name);
                if (expected == expected_shard.end())
                    throw std::runtime_error("tensor '" + name + "' exists in a shard but not in the checkpoint index");
                if (expected->second != s)
                    throw std::runtime_error("tensor '" + name + "' is stored in the wrong shard");
                if (!tensors_.emplace(name, TensorLocation{s, entry.second}).second)
                    throw std::runtime_error("tensor appears in multiple shards: " + name);
            }
        }
        for (const auto &entry : expected_shard)
            if (tensors_.find(entry.first) == tensors_.end())
                throw std::runtime_error("indexed tensor is missing from its shard: " + entry.first);
        if (actual_total != expected_total)
            throw std::runtime_error("checkpoint total_size mismatch: expected " + std::to_string(expected_total) +
                                     ", got " + std::to_string(actual_total));
        is_sharded_ = true;
    }

    bool SafetensorsCheckpoint::contains(std::string_view name) const { return tensors_.count(std::string(name)) != 0; }

    const SafetensorsTensorInfo &SafetensorsCheckpoint::tensor_info(std::string_view name) const
    {
        const auto it = tensors_.find(std::string(name));
        if (it == tensors_.end())
            throw std::out_of_range("checkpoint tensor not found: " + std::string(name));
        return it->second.info;
    }

    Tensor SafetensorsCheckpoint::load(std::string_view name, Device target_device) const
    {
        const auto it = tensors_.find(std::string(name));
        if (it == tensors_.end())
            throw std::out_of_range("checkpoint tensor not found: " + std::string(name));
        SafetensorsLoader loader{shard_paths_.at(it->second.shard_index)};
        if (!loader.metadata().contains(name) || !same_record(loader.metadata().tensor(name), it->second.info))
            throw std::runtime_error("checkpoint changed while loading tensor: " + std::string(name));
        return loader.load(name, target_device);
    }

    std::vector<Tensor> SafetensorsCheckpoint::load_many(const std::vector<std::string> &names,
                                                         Device target_device) const
    {
        // one loader (and one pinned staging pair) per shard, results in the order asked
        struct Group
        {
            std::size_t shard_index;
            std::vector<std::string> names;
            std::vector<std::size_t> slots;
        };
        std::vector<Group> groups;
        std::unordered_map<std::size_t, std::size_t> group_of_shard;
        for (std::size_t i = 0; i < names.size(); ++i)
        {
            const auto it = tensors_.find(names[i]);
            if (it == tensors_.end())
                throw std::out_of_range("checkpoint tensor not found: " + names[i]);
            const std::size_t shard = it->second.shard_index;
            auto g = group_of_shard.find(shard);
            if (g == group_of_shard.end())
            {
                g = group_of_shard.emplace(shard, groups.size()).first;
                groups.push_back(Group{shard, {}, {}});
            }
            groups[g->second].names.push_back(names[i]);
            groups[g->second].slots.push_back(i);
        }
        std::vector<Tensor> ordered;
        std::vector<Tensor *> filled(names.size(), nullptr);
        std::vector<std::vector<Tensor>> loaded_groups;
        loaded_groups.reserve(groups.size());
        for (const Group &group : groups)
        {
            SafetensorsLoader loader{shard_paths_.at(group.shard_index)};
            for (const std::string &n : group.names)
                if (!loader.metadata().contains(n) || !same_record(loader.metadata().tensor(n), tensors_.at(n).info))
                    throw std::runtime_error("checkpoint changed while loading tensor: " + n);
            loaded_groups.push_back(loader.load_many(group.names, target_device));
            if (loaded_groups.back().size() != group.names.size())
                throw std::logic_error("SafetensorsLoader returned an unexpected tensor count");
            for (std::size_t j = 0; j < group.slots.size(); ++j)
                filled[group.slots[j]] = &loaded_groups.back()[j];
        }
        ordered.reserve(names.size());
        for (Tensor *t : filled)
        {
            if (t == nullptr)
                throw std::logic_error("checkpoint did not fill every output slot");
            ordered.push_back(std::move(*t));
        }
        return ordered;
    }
} // namespace qwen3
