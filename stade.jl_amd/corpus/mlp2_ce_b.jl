function initstacks_mlp2_ce_b()
    return nothing
end

function mlp2_ce_b(loss, lossb, x, xb, lab, w1, w1b, b1, b1b, w2, w2b, b2, b2b, h1, h1b, z, zb, i_b, i_in, i_h, i_out)
    s1 = 0.0
    s2 = 0.0
    se = 0.0
    s1b = 0.0
    s2b = 0.0
    seb = 0.0
    for idx = 1:i_b * i_h
        __icse_0 = idx - 1
        i_s = div(__icse_0, i_h) + 1
        i_j = mod(__icse_0, i_h) + 1
        s1 = b1[i_j]
        for i_k = 1:i_in
            s1 = s1 + w1[(i_k - 1) * i_h + i_j] * x[(i_s - 1) * i_in + i_k]
        end
        h1[(i_s - 1) * i_h + i_j] = tanh(s1)
    end
    for idx2 = 1:i_b * i_out
        __icse_1 = idx2 - 1
        i_s2 = div(__icse_1, i_out) + 1
        i_o = mod(__icse_1, i_out) + 1
        s2 = b2[i_o]
        for i_k2 = 1:i_h
            s2 = s2 + w2[(i_k2 - 1) * i_out + i_o] * h1[(i_s2 - 1) * i_h + i_k2]
        end
        z[(i_s2 - 1) * i_out + i_o] = s2
    end
    for i_s3 = 1:i_b
        se = 0.0
        for i_o2 = 1:i_out
            se = se + exp(z[(i_s3 - 1) * i_out + i_o2])
        end
        i_l = lab[i_s3]
        loss[1] = loss[1] + (log(se) - z[(i_s3 - 1) * i_out + i_l])
    end
    for i_s3 = i_b:-1:1
        se = 0.0
        for i_o2 = 1:i_out
            se = se + exp(z[(i_s3 - 1) * i_out + i_o2])
        end
        i_l = lab[i_s3]
        __cse_2 = lossb[1]
        seb = seb + (1.0 / se) * __cse_2
        __icse_3 = (i_s3 - 1) * i_out + i_l
        zb[__icse_3] = zb[__icse_3] + -__cse_2
        for i_o2 = i_out:-1:1
            __icse_4 = (i_s3 - 1) * i_out + i_o2
            zb[__icse_4] = zb[__icse_4] + exp(z[__icse_4]) * seb
        end
        seb = 0.0
    end
    for idx2 = i_b * i_out:-1:1
        __icse_5 = idx2 - 1
        i_s2 = div(__icse_5, i_out) + 1
        i_o = mod(__icse_5, i_out) + 1
        __icse_6 = (i_s2 - 1) * i_out + i_o
        __oldb_0 = zb[__icse_6]
        zb[__icse_6] = 0.0
        s2b = s2b + __oldb_0
        for i_k2 = i_h:-1:1
            __icse_7 = (i_k2 - 1) * i_out + i_o
            __icse_8 = (i_s2 - 1) * i_h + i_k2
            w2b[__icse_7] = w2b[__icse_7] + h1[__icse_8] * s2b
            h1b[__icse_8] = h1b[__icse_8] + w2[__icse_7] * s2b
        end
        __oldb_1 = s2b
        s2b = 0.0
        b2b[i_o] = b2b[i_o] + __oldb_1
    end
    for idx = i_b * i_h:-1:1
        __icse_9 = idx - 1
        i_s = div(__icse_9, i_h) + 1
        i_j = mod(__icse_9, i_h) + 1
        s1 = b1[i_j]
        for i_k = 1:i_in
            s1 = s1 + w1[(i_k - 1) * i_h + i_j] * x[(i_s - 1) * i_in + i_k]
        end
        __icse_10 = (i_s - 1) * i_h + i_j
        __oldb_2 = h1b[__icse_10]
        h1b[__icse_10] = 0.0
        s1b = s1b + (1.0 - tanh(s1) ^ 2) * __oldb_2
        for i_k = i_in:-1:1
            __icse_11 = (i_k - 1) * i_h + i_j
            __icse_12 = (i_s - 1) * i_in + i_k
            w1b[__icse_11] = w1b[__icse_11] + x[__icse_12] * s1b
            xb[__icse_12] = xb[__icse_12] + w1[__icse_11] * s1b
        end
        __oldb_3 = s1b
        s1b = 0.0
        b1b[i_j] = b1b[i_j] + __oldb_3
    end
    return nothing
end

function mlp2_ce(loss, x, lab, w1, b1, w2, b2, h1, z, i_b, i_in, i_h, i_out)
    # hidden layer: one iteration per (sample, unit); the feature sum is carried (rule 1)
    for idx = 1:i_b * i_h
        i_s = div(idx - 1, i_h) + 1
        i_j = mod(idx - 1, i_h) + 1
        s1 = b1[i_j]
        for i_k = 1:i_in
            s1 = s1 + w1[(i_k - 1) * i_h + i_j] * x[(i_s - 1) * i_in + i_k]
        end
        h1[(i_s - 1) * i_h + i_j] = tanh(s1)
    end
    # output layer: one iteration per (sample, class)
    for idx2 = 1:i_b * i_out
        i_s2 = div(idx2 - 1, i_out) + 1
        i_o = mod(idx2 - 1, i_out) + 1
        s2 = b2[i_o]
        for i_k2 = 1:i_h
            s2 = s2 + w2[(i_k2 - 1) * i_out + i_o] * h1[(i_s2 - 1) * i_h + i_k2]
        end
        z[(i_s2 - 1) * i_out + i_o] = s2
    end
    # softmax cross-entropy of each sample, summed over the batch
    for i_s3 = 1:i_b
        se = 0.0
        for i_o2 = 1:i_out
            se = se + exp(z[(i_s3 - 1) * i_out + i_o2])
        end
        i_l = lab[i_s3]
        loss[1] = loss[1] + (log(se) - z[(i_s3 - 1) * i_out + i_l])
    end
    return nothing
end
